// bnn_kernel_abi.cpp - the reference's batch-1 kernel entry points
// (csrc/bnn_model.h:7-23, csrc/bnn_conv.c:50,80, and the v3 kernels of
// csrc/bnn_model_react.h:18-53) backed by the GPU.
//
// Same names, argument order and layouts as the reference, host pointers in
// and out, synchronous.  Each call stages its arrays through device memory,
// runs the kernel and copies the result back; on any HIP error it prints the
// error and exits, as the reference does on its own failures.  The 3x3 /
// pad 1 / stride 1 shapes of the UNet go through the engine's own kernels;
// other shapes through general kernels with the same arithmetic.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <memory>
#include <vector>

#include "bnn_kernels.h"
#include "bnn_model.h"
#include "bnn_model_react.h"

using namespace bnn;

namespace {

void check(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
    exit(1);
  }
}

// device buffer that lives for one call
struct Buf {
  void* p = nullptr;
  explicit Buf(size_t bytes) { check(hipMalloc(&p, bytes ? bytes : 4), "hipMalloc"); }
  ~Buf() { (void)hipFree(p); }
  template <class T>
  T* as() const { return (T*)p; }
};

Buf* up(const void* host, size_t bytes) {
  Buf* b = new Buf(bytes);
  if (bytes) check(hipMemcpy(b->p, host, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
  return b;
}
void down(void* host, const Buf& b, size_t bytes) {
  check(hipDeviceSynchronize(), "kernel");
  if (bytes) check(hipMemcpy(host, b.p, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
}
int out_dim(int n, int k, int pad, int stride) { return (n + 2 * pad - k) / stride + 1; }

// kidx sign bits -> [ceil(Cin/32)][coutp][taps] channel-per-tap words
std::vector<uint32_t> chan_words(const uint64_t* packed, int cin, int cout, int taps, int coutp) {
  const int nw = (cin * taps + 63) / 64, cw = (cin + 31) >> 5;
  std::vector<uint32_t> wt((size_t)cw * coutp * taps, 0u);
  for (int co = 0; co < cout; ++co)
    for (int ci = 0; ci < cin; ++ci)
      for (int t = 0; t < taps; ++t) {
        const int k = ci * taps + t;
        if ((packed[(size_t)co * nw + (k >> 6)] >> (k & 63)) & 1ull)
          wt[((size_t)(ci >> 5) * coutp + co) * taps + t] |= 1u << (ci & 31);
      }
  return wt;
}

// All three reference bconv kernels return the same integers
// (csrc/bnn_conv.c:5-15): an activation > 0 is bit 1, anything else bit 0.
void bconv_gpu(const int8_t* a, const uint64_t* packed_w, int32_t* P, int Cin, int H, int W, int Cout,
               int kh, int kw, int pad, int stride) {
  const int Ho = out_dim(H, kh, pad, stride), Wo = out_dim(W, kw, pad, stride);
  if (Ho <= 0 || Wo <= 0 || Cout <= 0) return;
  const int cw = (Cin + 31) >> 5;
  std::unique_ptr<Buf> da(up(a, (size_t)Cin * H * W));
  Buf act((size_t)H * W * cw * 4), dP((size_t)Cout * Ho * Wo * 4);
  check(launch_pack_act(da->as<int8_t>(), act.as<uint32_t>(), 1, Cin, H, W, 0), "pack");
  const bool fast = kh == 3 && kw == 3 && pad == 1 && stride == 1;
  const int coutp = fast ? (Cout + 31) & ~31 : Cout;
  std::vector<uint32_t> wt = chan_words(packed_w, Cin, Cout, kh * kw, coutp);
  std::unique_ptr<Buf> dw(up(wt.data(), wt.size() * 4));
  if (fast) {
    BconvArgs x{};
    x.in0 = act.as<uint32_t>(); x.cw0 = cw; x.N = 1; x.H = H; x.W = W; x.cin = Cin; x.cout = Cout;
    x.wt = dw->as<uint32_t>(); x.P = dP.as<int32_t>();
    check(launch_bconv(x, EPI_P, 1, Cout > 8 ? 32 : 8, false, 0), "bconv");
  } else {
    check(launch_bconv_generic(act.as<uint32_t>(), dw->as<uint32_t>(), dP.as<int32_t>(), Cin, H, W, Cout, kh, kw,
                               pad, stride, 0),
          "bconv");
  }
  down(P, dP, (size_t)Cout * Ho * Wo * 4);
}

}  // namespace

extern "C" {

void bconv_xnor(const int8_t* a, const uint64_t* packed_w, int32_t* P, int Cin, int H, int W, int Cout, int kh,
                int kw, int pad, int stride) {
  bconv_gpu(a, packed_w, P, Cin, H, W, Cout, kh, kw, pad, stride);
}
void bconv_xnor_packed(const int8_t* a, const uint64_t* packed_w, int32_t* P, int Cin, int H, int W, int Cout,
                       int kh, int kw, int pad, int stride) {
  bconv_gpu(a, packed_w, P, Cin, H, W, Cout, kh, kw, pad, stride);
}
void bconv_dispatch(const int8_t* a, const uint64_t* packed_w, int32_t* P, int Cin, int H, int W, int Cout,
                    int kh, int kw, int pad, int stride) {
  bconv_gpu(a, packed_w, P, Cin, H, W, Cout, kh, kw, pad, stride);
}

void bconv_naive_int(const int8_t* a, const int8_t* wsign, int32_t* P, int Cin, int H, int W, int Cout, int kh,
                     int kw, int pad, int stride) {
  const int Ho = out_dim(H, kh, pad, stride), Wo = out_dim(W, kw, pad, stride);
  if (Ho <= 0 || Wo <= 0 || Cout <= 0) return;
  std::unique_ptr<Buf> da(up(a, (size_t)Cin * H * W)), dw(up(wsign, (size_t)Cout * Cin * kh * kw));
  Buf dP((size_t)Cout * Ho * Wo * 4);
  check(launch_bconv_naive(da->as<int8_t>(), dw->as<int8_t>(), dP.as<int32_t>(), Cin, H, W, Cout, kh, kw, pad,
                           stride, 0),
        "bconv_naive");
  down(P, dP, (size_t)Cout * Ho * Wo * 4);
}

void pack_weights(const int8_t* wsign, uint64_t* packed, int Cout, int Cin, int kh, int kw) {
  const int K = Cin * kh * kw, nw = (K + 63) / 64;
  memset(packed, 0, (size_t)Cout * nw * 8);
  for (int co = 0; co < Cout; ++co)
    for (int k = 0; k < K; ++k)
      if (wsign[(size_t)co * K + k] > 0) packed[(size_t)co * nw + (k >> 6)] |= 1ull << (k & 63);
}

void conv_realin_naive(const float* x, const int8_t* wsign, const float* alpha, float* out, int Cin, int H, int W,
                       int Cout, int kh, int kw, int pad, int stride) {
  const int Ho = out_dim(H, kh, pad, stride), Wo = out_dim(W, kw, pad, stride);
  if (Ho <= 0 || Wo <= 0 || Cout <= 0) return;
  std::unique_ptr<Buf> dx(up(x, (size_t)Cin * H * W * 4));
  Buf dout((size_t)Cout * Ho * Wo * 4);
  const bool fast = kh == 3 && kw == 3 && pad == 1 && stride == 1;
  if (fast) {
    const int tot = (Cout + 31) / 32 * 32;
    std::vector<float> al(tot, 0.0f);
    std::copy(alpha, alpha + Cout, al.begin());
    std::unique_ptr<Buf> dw, dal(up(al.data(), al.size() * 4));
    RealArgs r{};
    if (real_conv_signs_only(wsign, Cout, Cin)) {
      std::vector<uint64_t> wm(real_conv_masks_len(Cout, Cin));
      real_conv_masks(wsign, Cout, Cin, wm.data());
      dw.reset(up(wm.data(), wm.size() * 8));
      r.wm = dw->as<uint64_t>();
    } else {
      std::vector<float> w(real_conv_weights_len(Cout, Cin));
      real_conv_weights(wsign, Cout, Cin, w.data());
      dw.reset(up(w.data(), w.size() * 4));
      r.w = dw->as<float>();
    }
    r.x = dx->as<float>();
    r.alpha = dal->as<float>();
    r.N = 1; r.H = H; r.W = W; r.cin = Cin; r.cout = Cout;
    r.f32 = dout.as<float>();
    check(launch_real(r, 0), "conv_realin");
  } else {
    std::vector<float> w((size_t)Cout * kh * kw * Cin);
    for (int co = 0; co < Cout; ++co)
      for (int ci = 0; ci < Cin; ++ci)
        for (int t = 0; t < kh * kw; ++t)
          w[((size_t)co * kh * kw + t) * Cin + ci] = (float)wsign[((size_t)co * Cin + ci) * kh * kw + t];
    std::unique_ptr<Buf> dw(up(w.data(), w.size() * 4)), dal(up(alpha, (size_t)Cout * 4));
    check(launch_real_generic(dx->as<float>(), dw->as<float>(), dal->as<float>(), dout.as<float>(), Cin, H, W, Cout,
                              kh, kw, pad, stride, 0),
          "conv_realin");
  }
  down(out, dout, (size_t)Cout * Ho * Wo * 4);
}

void maxpool_P(const int32_t* P, int32_t* Pout, int C, int H, int W, int k, int stride) {
  const int Ho = (H - k) / stride + 1, Wo = (W - k) / stride + 1;
  if (Ho <= 0 || Wo <= 0 || C <= 0) return;
  std::unique_ptr<Buf> dP(up(P, (size_t)C * H * W * 4));
  Buf dO((size_t)C * Ho * Wo * 4);
  check(launch_maxpool(dP->as<int32_t>(), dO.as<int32_t>(), C, H, W, k, stride, 0), "maxpool");
  down(Pout, dO, (size_t)C * Ho * Wo * 4);
}

void apply_fold_int(const int32_t* P, int8_t* out, int C, int H, int W, const int32_t* type, const int32_t* t,
                    const int32_t* lo, const int32_t* hi) {
  const size_t n = (size_t)C * H * W;
  if (!n) return;
  std::unique_ptr<Buf> dP(up(P, n * 4)), dty(up(type, C * 4)), dt(up(t, C * 4)), dlo(up(lo, C * 4)),
      dhi(up(hi, C * 4));
  Buf dO(n);
  check(launch_fold_int(dP->as<int32_t>(), dO.as<int8_t>(), C, H * W, dty->as<int32_t>(), dt->as<int32_t>(),
                        dlo->as<int32_t>(), dhi->as<int32_t>(), 0),
        "fold_int");
  down(out, dO, n);
}

void apply_fold_real(const float* x, int8_t* out, int C, int H, int W, const float* A, const float* B,
                     const float* slope, const float* rsign) {
  const size_t n = (size_t)C * H * W;
  if (!n) return;
  std::unique_ptr<Buf> dx(up(x, n * 4)), dA(up(A, C * 4)), dB(up(B, C * 4)), ds(up(slope, C * 4)),
      dr(up(rsign, C * 4));
  Buf dO(n);
  check(launch_fold_real(dx->as<float>(), dO.as<int8_t>(), C, H * W, dA->as<float>(), dB->as<float>(),
                         ds->as<float>(), dr->as<float>(), 0),
        "fold_real");
  down(out, dO, n);
}

void head_1x1(const float* a, const float* Wt, const float* bias, float* logits, int Cin, int H, int W_, int Cout) {
  const size_t hw = (size_t)H * W_;
  if (!hw || Cout <= 0) return;
  std::unique_ptr<Buf> da(up(a, (size_t)Cin * hw * 4)), dw(up(Wt, (size_t)Cout * Cin * 4)),
      db(up(bias, (size_t)Cout * 4));
  Buf dO((size_t)Cout * hw * 4);
  check(launch_head(da->as<float>(), dw->as<float>(), db->as<float>(), dO.as<float>(), Cin, (int)hw, Cout, 0),
        "head");
  down(logits, dO, (size_t)Cout * hw * 4);
}

// ---------------------------------------------------------------- v3 ----
// csrc/bnn_react_ops.c:36-70 (form 0) and csrc/bnn_react_epi.c:11-77 (form 1)
static void react_epi(const void* acc, int kind, size_t esz, const float* res, float* out, int C, int H, int W,
                      const float* A, const float* B, const float* move1, const float* prelu_w, int form) {
  const size_t n = (size_t)C * H * W;
  if (!n) return;
  std::unique_ptr<Buf> dacc(up(acc, n * esz)), dres(up(res, n * 4)), dA(up(A, C * 4)), dB(up(B, C * 4)),
      dm(up(move1, C * 4)), dw(up(prelu_w, C * 4));
  Buf dO(n * 4);
  check(launch_react_epi(dacc->p, kind, dres->as<float>(), dO.as<float>(), C, (long)H * W, dA->as<float>(),
                         dB->as<float>(), dm->as<float>(), dw->as<float>(), form, 0),
        "react_epilogue");
  down(out, dO, n * 4);
}

void react_epilogue_int(const int32_t* P, const float* res, float* out, int C, int H, int W, const float* A,
                        const float* B, const float* move1, const float* prelu_w) {
  react_epi(P, 0, 4, res, out, C, H, W, A, B, move1, prelu_w, 0);
}
void react_epilogue_real(const float* cin, const float* res, float* out, int C, int H, int W, const float* A,
                         const float* B, const float* move1, const float* prelu_w) {
  react_epi(cin, 2, 4, res, out, C, H, W, A, B, move1, prelu_w, 0);
}
void react_epilogue_int_v2(const int32_t* P, const float* res, float* out, int C, int H, int W, const float* A,
                           const float* B, const float* move1, const float* prelu_w) {
  react_epi(P, 0, 4, res, out, C, H, W, A, B, move1, prelu_w, 1);
}
void react_epilogue_int_i16(const int16_t* P, const float* res, float* out, int C, int H, int W, const float* A,
                            const float* B, const float* move1, const float* prelu_w) {
  react_epi(P, 1, 2, res, out, C, H, W, A, B, move1, prelu_w, 1);
}
void react_epilogue_real_v2(const float* cin, const float* res, float* out, int C, int H, int W, const float* A,
                            const float* B, const float* move1, const float* prelu_w) {
  react_epi(cin, 2, 4, res, out, C, H, W, A, B, move1, prelu_w, 1);
}

void react_tap(const float* x, int8_t* out, int C, int H, int W, const float* rsign) {
  const size_t n = (size_t)C * H * W;
  if (!n) return;
  std::unique_ptr<Buf> dx(up(x, n * 4)), dr(up(rsign, C * 4));
  Buf dO(n);
  check(launch_react_tap(dx->as<float>(), dO.as<int8_t>(), C, (long)H * W, dr->as<float>(), 0), "react_tap");
  down(out, dO, n);
}

void maxpool_real(const float* x, float* out, int C, int H, int W, int k, int stride) {
  if (k <= 0 || stride <= 0 || H < k || W < k || C <= 0) return;
  const int Ho = (H - k) / stride + 1, Wo = (W - k) / stride + 1;
  std::unique_ptr<Buf> dx(up(x, (size_t)C * H * W * 4));
  Buf dO((size_t)C * Ho * Wo * 4);
  check(launch_maxpool_real(dx->as<float>(), dO.as<float>(), C, H, W, k, stride, 0), "maxpool_real");
  down(out, dO, (size_t)C * Ho * Wo * 4);
}
// 2x2 / stride 2 only; any other window leaves out untouched (csrc/bnn_react_opt.c:48)
void maxpool_real_v2(const float* x, float* out, int C, int H, int W, int k, int stride) {
  if (k != 2 || stride != 2) return;
  maxpool_real(x, out, C, H, W, 2, 2);
}
void maxpool_P_v2(const int32_t* x, int32_t* out, int C, int H, int W, int k, int stride) {
  if (k != 2 || stride != 2) return;
  maxpool_P(x, out, C, H, W, 2, 2);
}
void maxpool_P_i16(const int16_t* x, int16_t* out, int C, int H, int W, int k, int stride) {
  if (k != 2 || stride != 2 || H < 2 || W < 2 || C <= 0) return;
  const int Ho = H / 2, Wo = W / 2;
  std::vector<int32_t> xi((size_t)C * H * W), oi((size_t)C * Ho * Wo);
  for (size_t i = 0; i < xi.size(); ++i) xi[i] = x[i];
  maxpool_P(xi.data(), oi.data(), C, H, W, 2, 2);
  for (size_t i = 0; i < oi.size(); ++i) out[i] = (int16_t)oi[i];
}

// one chain over ci from 0 per output: react_proj_blk for Cout % 8 == 0
// (csrc/bnn_realin_blk.h:39-83, which exits otherwise), react_proj_1x1
// (csrc/bnn_react_ops.c:117-133) for any Cout; both on the matrix cores
static void proj_gpu(const float* x, const float* Wm, float* out, int Cin, int H, int W, int Cout) {
  const size_t hw = (size_t)H * W;
  if (!hw || Cout <= 0) return;
  std::vector<float> lanes(react_pw_lanes_len(Cout, Cin));
  react_pw_lanes(Wm, Cout, Cin, lanes.data());
  std::unique_ptr<Buf> dx(up(x, (size_t)Cin * hw * 4)), dw(up(lanes.data(), lanes.size() * 4));
  Buf dO((size_t)Cout * hw * 4);
  ProjArgs p{};
  p.x0 = dx->as<float>(); p.c0 = Cin; p.cin = Cin; p.cout = Cout;
  p.N = 1; p.H = H; p.W = W; p.w = dw->as<float>(); p.out = dO.as<float>();
  check(launch_proj(p, 0), "react_proj");
  down(out, dO, (size_t)Cout * hw * 4);
}
void react_proj_1x1(const float* x, const float* Wm, float* out, int Cin, int H, int W, int Cout) {
  proj_gpu(x, Wm, out, Cin, H, W, Cout);
}
void react_proj_blk(const float* x, const float* Wm, float* out, int Cin, int H, int W, int Cout) {
  if (Cout % 8) {
    fprintf(stderr, "proj_blk: Cout %% CB != 0\n");
    exit(1);
  }
  proj_gpu(x, Wm, out, Cin, H, W, Cout);
}

void react_conv3_blk(const float* x, const int8_t* wsign, const float* alpha, float* out, int Cin, int H, int W,
                     int Cout) {
  if (Cout % 8) {
    fprintf(stderr, "conv3_blk: Cout %% CB != 0\n");
    exit(1);
  }
  const size_t hw = (size_t)H * W;
  if (!hw || Cout <= 0) return;
  std::unique_ptr<Buf> dx(up(x, (size_t)Cin * hw * 4)), dw(up(wsign, (size_t)Cout * Cin * 9)),
      da(up(alpha, (size_t)Cout * 4));
  Buf dO((size_t)Cout * hw * 4);
  check(launch_conv3_chain(dx->as<float>(), dw->as<int8_t>(), da->as<float>(), dO.as<float>(), Cin, H, W, Cout, 0),
        "react_conv3");
  down(out, dO, (size_t)Cout * hw * 4);
}

// the register-tiled binary convs give the integers of every other bconv
// kernel (csrc/bnn_bconv_blk.h:30-156), int16 storage included
void bconv_blk_b4p4(const int8_t* a, const uint64_t* packed_w, int32_t* P, int Cin, int H, int W, int Cout, int kh,
                    int kw, int pad, int stride) {
  bconv_gpu(a, packed_w, P, Cin, H, W, Cout, kh, kw, pad, stride);
}
void bconv_blk_b4p4_i16(const int8_t* a, const uint64_t* packed_w, int16_t* P, int Cin, int H, int W, int Cout,
                        int kh, int kw, int pad, int stride) {
  const int Ho = out_dim(H, kh, pad, stride), Wo = out_dim(W, kw, pad, stride);
  if (Ho <= 0 || Wo <= 0 || Cout <= 0) return;
  std::vector<int32_t> Pi((size_t)Cout * Ho * Wo);
  bconv_gpu(a, packed_w, Pi.data(), Cin, H, W, Cout, kh, kw, pad, stride);
  for (size_t i = 0; i < Pi.size(); ++i) P[i] = (int16_t)Pi[i];
}

// bias, then channels in order, one fused step each: the same arithmetic as
// head_1x1 (csrc/bnn_react_opt.c:33-41 on x86)
void head_1x1_v2(const float* a, const float* Wt, const float* bias, float* logits, int Cin, int H, int W_,
                 int Cout) {
  head_1x1(a, Wt, bias, logits, Cin, H, W_, Cout);
}

}  // extern "C"
