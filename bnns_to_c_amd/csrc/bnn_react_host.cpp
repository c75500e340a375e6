// bnn_react_host.cpp - libbnn_hip.so host side of the v3 (ReActNet,
// real-highway) model: blob v3 parsing, device model, the batched forward
// and its debug / patch-wise / file variants, and the C ABI of
// include/bnn_model_react.h.
//
// Blob: python/bnn2c/blob_react.py:8-41, read with the checks of
// csrc/bnn_model_react.c:44-135.  Forward: csrc/bnn_model_react.c:6-14,
// 190-274, 395-438, one kernel per fused stage over a batch of N
// independent patches:
//   enc1   launch_react_in: conv + projection + epilogue -> h1 and tap2 bits
//          (Cout % 8 != 0: launch_real's general-order conv, then
//          launch_react_in_tail for the projection, epilogue and tap)
//   unit 1 launch_proj (res), then the binary conv of the tap1 bits with the
//          RPReLU epilogue -> h1 and its tap2 bits
//   unit 2 the binary conv of the tap2 bits; down blocks: skip h and the
//          pooled down h in one epilogue, each with the bits of the tap that
//          reads it next; plain blocks: h2 and the bits of the next
//          decoder's tap on its upsample; dec1: the head.
// The highway lives in HBM as float planes [C][N*H*W]; binary activations as
// channel-packed words [N][H][W][ceil(C/32)] (bnn_kernels.h).  A tap is
// applied by the kernel that produces its input, with the consumer's rsign,
// so no stage reads the highway just to binarise it.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "bnn_host_internal.h"
#include "bnn_kernels.h"
#include "bnn_model.h"
#include "bnn_model_react.h"
#include "bnn_prof.h"

using namespace bnn;

namespace {

constexpr int TAG_BIN = 1, TAG_REAL = 2, TAG_HEAD = 4, TAG_PROJ = 5, TAG_EPI = 6, TAG_TAP = 7;

// ------------------------------------------------------------ blob reader
struct Reader {
  FILE* f;
  const char* path;
  int rc = BNN_OK;
  bool ok() const { return rc == BNN_OK; }
  void fail(const char* fmt, const char* what = "", int v = 0) {
    if (ok()) rc = set_err(BNN_EBLOB, fmt, what, v);
  }
  int i32() {
    int v = 0;
    if (ok() && fread(&v, 4, 1, f) != 1) fail("%sshort read", "");
    return ok() ? v : 0;
  }
  template <class T>
  T* arr(long long n) {
    if (!ok()) return nullptr;
    if (n < 0 || n > (1ll << 34)) { fail("%sbad record size", ""); return nullptr; }
    T* p = (T*)malloc(n ? (size_t)n * sizeof(T) : 1);
    if (!p) { fail("%sout of memory", ""); return nullptr; }
    if (n && fread(p, sizeof(T), (size_t)n, f) != (size_t)n) {
      free(p);
      fail("%sshort read", "");
      return nullptr;
    }
    return p;
  }
};

void read_conv(Reader& r, ConvR* c) {
  memset(c, 0, sizeof *c);
  c->tag = r.i32();
  c->Cout = r.i32(); c->Cin = r.i32(); c->kh = r.i32(); c->kw = r.i32();
  c->pad = r.i32(); c->stride = r.i32();
  if (!r.ok()) return;
  if (c->Cout < 0 || c->Cin < 0 || c->kh < 0 || c->kw < 0) return r.fail("%snegative conv dims");
  if (c->tag == TAG_BIN) {
    c->nwords = r.i32();
    c->packed = r.arr<uint64_t>((long long)c->Cout * c->nwords);
  } else if (c->tag == TAG_REAL) {
    c->wsign = r.arr<int8_t>((long long)c->Cout * c->Cin * c->kh * c->kw);
    c->alpha = r.arr<float>(c->Cout);
  } else {
    r.fail("bad conv tag %s%d", "", c->tag);
  }
}

void read_proj(Reader& r, ProjR* p) {
  memset(p, 0, sizeof *p);
  const int tag = r.i32();
  if (r.ok() && tag != TAG_PROJ) return r.fail("bad proj tag %s%d", "", tag);
  p->Cout = r.i32(); p->Cin = r.i32();
  if (r.ok() && (p->Cout < 0 || p->Cin < 0)) return r.fail("%snegative proj dims");
  p->W = r.arr<float>((long long)p->Cout * p->Cin);
}

void read_epi(Reader& r, EpiR* e) {
  memset(e, 0, sizeof *e);
  const int tag = r.i32();
  if (r.ok() && tag != TAG_EPI) return r.fail("bad epi tag %s%d", "", tag);
  e->kind = r.i32(); e->C = r.i32();
  e->A = r.arr<float>(e->C); e->B = r.arr<float>(e->C);
  e->move1 = r.arr<float>(e->C); e->prelu_w = r.arr<float>(e->C);
}

void read_tap(Reader& r, TapR* t) {
  memset(t, 0, sizeof *t);
  const int tag = r.i32();
  if (r.ok() && tag != TAG_TAP) return r.fail("bad tap tag %s%d", "", tag);
  t->C = r.i32();
  t->rsign = r.arr<float>(t->C);
}

// one block and the loader's structural checks (csrc/bnn_model_react.c:86-106)
void read_block(Reader& r, BlockR* b, int is_down, int input_real) {
  memset(b, 0, sizeof *b);
  b->is_down = is_down; b->input_real = input_real;
  if (!input_real) read_tap(r, &b->tap1);
  read_conv(r, &b->conv1); read_proj(r, &b->proj1); read_epi(r, &b->epi1);
  read_tap(r, &b->tap2); read_conv(r, &b->conv2); read_epi(r, &b->epi_a);
  if (is_down) read_epi(r, &b->epi_b);
  if (!r.ok()) return;
  auto check = [&](bool ok, const char* what) {
    if (!ok) r.fail("blob layout mismatch: %s", what);
  };
  check(b->conv1.tag == (input_real ? TAG_REAL : TAG_BIN), "conv1 tag");
  check(b->conv2.tag == TAG_BIN, "conv2 tag");
  check(b->proj1.Cin == b->conv1.Cin && b->proj1.Cout == b->conv1.Cout, "proj1 dims");
  check(input_real || b->tap1.C == b->conv1.Cin, "tap1 channels");
  check(b->tap2.C == b->conv2.Cin, "tap2 channels");
  check(b->epi1.C == b->conv1.Cout && b->epi1.kind == (input_real ? 1 : 0), "epi1");
  check(b->epi_a.C == b->conv2.Cout && b->epi_a.kind == 0, "epi_a");
  check(!is_down || (b->epi_b.C == b->conv2.Cout && b->epi_b.kind == 0), "epi_b");
}

void free_block(BlockR* b) {
  free(b->tap1.rsign); free(b->tap2.rsign);
  free(b->conv1.packed); free(b->conv1.wsign); free(b->conv1.alpha);
  free(b->conv2.packed); free(b->conv2.wsign); free(b->conv2.alpha);
  free(b->proj1.W);
  for (EpiR* e : {&b->epi1, &b->epi_a, &b->epi_b}) { free(e->A); free(e->B); free(e->move1); free(e->prelu_w); }
}

void free_host(ModelR* m) {
  if (!m) return;
  for (int i = 0; i < 4; ++i) { free_block(&m->enc[i]); free_block(&m->dec[i]); }
  free_block(&m->bott);
  free(m->head_W); free(m->head_bias);
  free(m);
}

int parse_blob(const char* path, ModelR** out) {
  *out = nullptr;
  FILE* f = fopen(path, "rb");
  if (!f) return set_err(BNN_EBLOB, "cannot open %s", path);
  Reader r{f, path};
  ModelR* m = (ModelR*)calloc(1, sizeof(ModelR));
  char magic[4] = {0};
  if (fread(magic, 1, 4, f) != 4 || memcmp(magic, "BNNC", 4) != 0) r.fail("%sbad magic");
  m->version = r.i32();
  if (r.ok() && m->version != 3) r.fail("blob version %s%d, this engine reads v3 (ReActNet)", "", m->version);
  m->base_channels = r.i32(); m->n_bands = r.i32(); m->n_classes = r.i32(); m->upsampler = r.i32();
  if (r.ok() && m->upsampler != 0) r.fail("%sonly nearest upsampler supported");
  for (int i = 0; i < 4; ++i) read_block(r, &m->enc[i], 1, i == 0);
  read_block(r, &m->bott, 0, 0);
  for (int i = 0; i < 4; ++i) read_block(r, &m->dec[i], 0, 0);
  const int tag = r.i32();
  if (r.ok() && tag != TAG_HEAD) r.fail("bad head tag %s%d", "", tag);
  m->head_Cout = r.i32(); m->head_Cin = r.i32();
  if (r.ok() && (m->head_Cout < 0 || m->head_Cin < 0)) r.fail("%snegative head dims");
  m->head_W = r.arr<float>((long long)m->head_Cout * m->head_Cin);
  m->head_bias = r.arr<float>(m->head_Cout);
  char extra;
  if (r.ok() && fread(&extra, 1, 1, f) != 0) r.fail("%strailing bytes in blob");
  fclose(f);
  if (!r.ok()) { free_host(m); return r.rc; }
  *out = m;
  return BNN_OK;
}

// What this engine runs beyond the reader's checks: the widths chain as the
// forward uses them (the reference trusts them), every conv is 3x3 / pad 1
// / stride 1 (the reference's binary path exits otherwise,
// csrc/bnn_model_react.c:146-151), and an enc1.conv1 on the reference's
// register-blocked path (Cout % 8 == 0, csrc/bnn_model_react.c:152-158)
// has +-1 signs (its matrix-core kernel holds them as lane masks).  With
// Cout % 8 != 0 the reference's general conv runs instead, here the v1
// first-conv kernels, which take any int8 signs.
int validate(const ModelR* m) {
  auto k3 = [](const ConvR& c) {
    return c.kh == 3 && c.kw == 3 && c.pad == 1 && c.stride == 1 &&
           (c.tag != TAG_BIN || c.nwords == (c.Cin * 9 + 63) / 64);
  };
  int prev = m->n_bands, skipC[4];
  for (int i = 0; i < 4; ++i) {
    const BlockR& b = m->enc[i];
    if (b.conv1.Cin != prev || b.conv2.Cin != b.conv1.Cout || b.conv2.Cout != b.conv1.Cout)
      return set_err(BNN_EBLOB, "enc%d: channel widths do not chain", i + 1);
    if (!k3(b.conv1) || !k3(b.conv2)) return set_err(BNN_EBLOB, "enc%d: only 3x3/pad 1/stride 1 convs", i + 1);
    skipC[i] = b.conv2.Cout;
    prev = b.conv2.Cout;
  }
  const ConvR& r = m->enc[0].conv1;
  if (r.Cout % 8 == 0 && !real_conv_signs_only(r.wsign, r.Cout, r.Cin))
    return set_err(BNN_EBLOB, "enc1.conv1: signs must be +-1 when Cout is a multiple of 8");
  const BlockR& bt = m->bott;
  if (bt.conv1.Cin != prev || bt.conv2.Cin != bt.conv1.Cout || bt.conv2.Cout != bt.conv1.Cout)
    return set_err(BNN_EBLOB, "bottleneck: channel widths do not chain");
  if (!k3(bt.conv1) || !k3(bt.conv2)) return set_err(BNN_EBLOB, "bottleneck: only 3x3/pad 1/stride 1 convs");
  prev = bt.conv2.Cout;
  for (int i = 0; i < 4; ++i) {
    const BlockR& b = m->dec[i];
    if (b.conv1.Cin != skipC[3 - i] + prev || b.conv2.Cin != b.conv1.Cout || b.conv2.Cout != b.conv1.Cout)
      return set_err(BNN_EBLOB, "dec%d: channel widths do not chain", 4 - i);
    if (!k3(b.conv1) || !k3(b.conv2)) return set_err(BNN_EBLOB, "dec%d: only 3x3/pad 1/stride 1 convs", 4 - i);
    prev = b.conv2.Cout;
  }
  if (m->head_Cin != prev || m->head_Cout != m->n_classes)
    return set_err(BNN_EBLOB, "head %dx%d does not match dec1 (%d) / n_classes (%d)", m->head_Cout, m->head_Cin,
                   prev, m->n_classes);
  if (m->n_bands <= 0 || m->n_classes <= 0) return set_err(BNN_EBLOB, "bad n_bands / n_classes");
  return BNN_OK;
}

// ------------------------------------------------------------ device model
struct DevEpi {
  float *A = nullptr, *B = nullptr, *W = nullptr;  // B = B + move1, padded to 32
};

struct DevBlock {
  int cin = 0, cout = 0, cs = 0, cw0 = 0, cw1 = 0;
  uint32_t *w1 = nullptr, *w2 = nullptr;  // binary conv words (w1 unused for enc1)
  int p1 = 0, p2 = 0;                      // w1 / w2 hold paired taps (inputs of at most 16 channels)
  float* pw = nullptr;                     // projection lanes (binary blocks)
  DevEpi e1, ea, eb;
  float *t1a = nullptr, *t1b = nullptr;    // tap1 rsign: skip part / upsampled part (decoders); t1a only otherwise
  float* t2 = nullptr;
};

struct RWorkspace {
  int N = 0, H = 0, W = 0;
  uint8_t* base = nullptr;
  size_t cap = 0;  // bytes at base
  float *h1[9] = {}, *res[9] = {}, *h2[9] = {}, *skip[4] = {}, *down[4] = {};
  uint32_t *a2[9] = {}, *skipb[4] = {}, *downb[4] = {}, *upb[9] = {};
};

struct Dumps {
  bool on = false;
  float *conv = nullptr, *proj = nullptr;  // enc1 [N][C][H][W]
  int32_t* P[18] = {};
  int32_t* P2[4] = {};
};

struct Scene {
  int sH, sW, pcols, prow0;
};

}  // namespace

struct BnnReactDevice {
  int device = 0;
  hipStream_t stream = nullptr;
  std::vector<void*> allocs;
  int rcin = 0, rcout = 0;
  uint64_t* rwm = nullptr;
  float *ralpha = nullptr, *rpw = nullptr;
  // enc1.conv1 with Cout % 8 != 0: the general-order conv (launch_real, lane
  // masks in rwm when every sign is +-1, else floats in rw) and the
  // projection as plain rows for launch_react_in_tail (rpw)
  bool rgen = false;
  float* rw = nullptr;
  DevBlock blk[9];  // enc1..4, bott, dec4..1
  float *hw = nullptr, *hb = nullptr;
  int ncls = 0;
  RWorkspace ws;
  float *stage_in = nullptr, *stage_out = nullptr;
  size_t stage_in_cap = 0, stage_out_cap = 0;
  // one strip of whole patch rows of a cube of 2 GiB or more, staged as a
  // sub-cube [nb][rows][W], and its map rows
  float *strip_in = nullptr, *strip_out = nullptr;
  size_t strip_in_cap = 0, strip_out_cap = 0;
  // pinned row strips of a streamed input file, filled in turn
  float* strip[2] = {nullptr, nullptr};
  hipEvent_t strip_done[2] = {nullptr, nullptr};
  // the second half of a large batch runs on this stream
  hipStream_t side = nullptr;
  hipEvent_t ev_fork = nullptr, ev_join = nullptr;
};

namespace {

template <class T>
int dev_upload(BnnReactDevice* D, T** dst, const T* src, size_t n) {
  void* p = nullptr;
  HIP_TRY(hipMalloc(&p, n ? n * sizeof(T) : 4));
  D->allocs.push_back(p);
  if (n) HIP_TRY(hipMemcpy(p, src, n * sizeof(T), hipMemcpyHostToDevice));
  *dst = (T*)p;
  return BNN_OK;
}

// a per-channel float array zero-padded to whole 32-channel words
int upload_pad(BnnReactDevice* D, float** dst, const float* src, int n, int off = 0) {
  std::vector<float> v((size_t)pad32(n), 0.0f);
  if (src) std::copy(src + off, src + off + n, v.begin());
  return dev_upload(D, dst, v.data(), v.size());
}

int upload_epi(BnnReactDevice* D, DevEpi* e, const EpiR& r) {
  std::vector<float> bm((size_t)r.C);
  for (int c = 0; c < r.C; ++c) bm[c] = r.B[c] + r.move1[c];  // one float add, as the reference hoists it
  int rc;
  if ((rc = upload_pad(D, &e->A, r.A, r.C))) return rc;
  if ((rc = upload_pad(D, &e->B, bm.data(), r.C))) return rc;
  return upload_pad(D, &e->W, r.prelu_w, r.C);
}

void release(BnnReactDevice* D) {
  if (!D) return;
  if (D->stream) (void)hipStreamSynchronize(D->stream);
  if (D->side) (void)hipStreamSynchronize(D->side);
  for (void* p : D->allocs) (void)hipFree(p);
  D->allocs.clear();
  if (D->ws.base) (void)hipFree(D->ws.base);
  if (D->stage_in) (void)hipFree(D->stage_in);
  if (D->strip_in) (void)hipFree(D->strip_in);
  if (D->strip_out) (void)hipFree(D->strip_out);
  if (D->stage_out) (void)hipFree(D->stage_out);
  for (int k = 0; k < 2; ++k) {
    if (D->strip[k]) (void)hipHostFree(D->strip[k]);
    if (D->strip_done[k]) (void)hipEventDestroy(D->strip_done[k]);
    D->strip[k] = nullptr;
    D->strip_done[k] = nullptr;
  }
  if (D->ev_fork) (void)hipEventDestroy(D->ev_fork);
  if (D->ev_join) (void)hipEventDestroy(D->ev_join);
  if (D->side) (void)hipStreamDestroy(D->side);
  if (D->stream) (void)hipStreamDestroy(D->stream);
  D->stream = nullptr;
}

// block index: 0..3 enc1..4, 4 bott, 5..8 dec4..dec1
const BlockR& block_of(const ModelR* m, int k) { return k < 4 ? m->enc[k] : k == 4 ? m->bott : m->dec[k - 5]; }

int build_device(ModelR* m) {
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
    return set_err(BNN_EHIP, "no HIP device visible: libbnn_hip runs the forward on the GPU only");
  BnnReactDevice* D = new BnnReactDevice();
  m->dev = D;
  HIP_TRY(hipGetDevice(&D->device));
  HIP_TRY(hipStreamCreateWithFlags(&D->stream, hipStreamNonBlocking));
  int rc;
  {
    const ConvR& c = m->enc[0].conv1;
    D->rcin = c.Cin; D->rcout = c.Cout;
    D->rgen = c.Cout % 8 != 0;
    if (!D->rgen || real_conv_signs_only(c.wsign, c.Cout, c.Cin)) {
      std::vector<uint64_t> wm(real_conv_masks_len(c.Cout, c.Cin));
      real_conv_masks(c.wsign, c.Cout, c.Cin, wm.data());
      if ((rc = dev_upload(D, &D->rwm, wm.data(), wm.size()))) return rc;
    } else {
      std::vector<float> w(real_conv_weights_len(c.Cout, c.Cin));
      real_conv_weights(c.wsign, c.Cout, c.Cin, w.data());
      if ((rc = dev_upload(D, &D->rw, w.data(), w.size()))) return rc;
    }
    if (D->rgen) {
      const int cp = (c.Cout + 15) / 16 * 16;
      std::vector<float> pw((size_t)cp * c.Cin, 0.0f);
      std::copy(m->enc[0].proj1.W, m->enc[0].proj1.W + (size_t)c.Cout * c.Cin, pw.begin());
      if ((rc = dev_upload(D, &D->rpw, pw.data(), pw.size()))) return rc;
    } else {
      std::vector<float> pw(react_proj_lanes_len(c.Cout, c.Cin));
      react_proj_lanes(m->enc[0].proj1.W, c.Cout, c.Cin, pw.data());
      if ((rc = dev_upload(D, &D->rpw, pw.data(), pw.size()))) return rc;
    }
    if ((rc = upload_pad(D, &D->ralpha, c.alpha, c.Cout))) return rc;
  }
  for (int k = 0; k < 9; ++k) {
    const BlockR& b = block_of(m, k);
    DevBlock& L = D->blk[k];
    L.cin = b.conv1.Cin; L.cout = b.conv1.Cout;
    L.cs = k >= 5 ? m->enc[8 - k].conv2.Cout : 0;  // the skip width of a decoder's concat
    L.cw0 = words(L.cs ? L.cs : L.cin);
    L.cw1 = L.cs ? words(L.cin - L.cs) : 0;
    if (!b.input_real) {
      std::vector<uint32_t> w = repack_bin(b.conv1.packed, L.cin, L.cout, 9, L.cs);
      L.p1 = (L.cs ? L.cs : L.cin) <= 16;
      if (L.p1) w = pair_taps(w, L.cout);
      if ((rc = dev_upload(D, &L.w1, w.data(), w.size()))) return rc;
      std::vector<float> pw(react_pw_lanes_len(L.cout, L.cin));
      react_pw_lanes(b.proj1.W, L.cout, L.cin, pw.data());
      if ((rc = dev_upload(D, &L.pw, pw.data(), pw.size()))) return rc;
      if ((rc = upload_pad(D, &L.t1a, b.tap1.rsign, L.cs ? L.cs : L.cin))) return rc;
      if (L.cs && (rc = upload_pad(D, &L.t1b, b.tap1.rsign, L.cin - L.cs, L.cs))) return rc;
    }
    std::vector<uint32_t> w2 = repack_bin(b.conv2.packed, b.conv2.Cin, b.conv2.Cout, 9, 0);
    L.p2 = b.conv2.Cin <= 16;
    if (L.p2) w2 = pair_taps(w2, b.conv2.Cout);
    if ((rc = dev_upload(D, &L.w2, w2.data(), w2.size()))) return rc;
    if ((rc = upload_pad(D, &L.t2, b.tap2.rsign, b.tap2.C))) return rc;
    if ((rc = upload_epi(D, &L.e1, b.epi1))) return rc;
    if ((rc = upload_epi(D, &L.ea, b.epi_a))) return rc;
    if (b.is_down && (rc = upload_epi(D, &L.eb, b.epi_b))) return rc;
  }
  D->ncls = m->head_Cout;
  if ((rc = dev_upload(D, &D->hw, m->head_W, (size_t)m->head_Cout * m->head_Cin))) return rc;
  if ((rc = dev_upload(D, &D->hb, m->head_bias, (size_t)m->head_Cout))) return rc;
  HIP_TRY(hipDeviceSynchronize());
  return BNN_OK;
}

// per-level spatial dims: level 0 = input, 1..4 after each pool
void level_dims(int H, int W, int* hs, int* wsz) {
  hs[0] = H; wsz[0] = W;
  for (int l = 1; l <= 4; ++l) { hs[l] = hs[l - 1] / 2; wsz[l] = wsz[l - 1] / 2; }
}
// level of block k's output
int level_of(int k) { return k < 4 ? k : k == 4 ? 4 : 8 - k; }

int ensure_ws(const ModelR* m, BnnReactDevice* D, RWorkspace& w, int N, int H, int W) {
  if (w.base && w.N >= N && w.H == H && w.W == W) return BNN_OK;
  int hs[5], wsz[5];
  level_dims(H, W, hs, wsz);
  std::vector<std::pair<void**, size_t>> plan;  // bytes
  auto px = [&](int lvl) { return (size_t)N * hs[lvl] * wsz[lvl]; };
  auto planes = [&](float** p, int lvl, int c) { plan.push_back({(void**)p, px(lvl) * c * 4}); };
  // bit buffers hold one more pixel: the pad pixel of a concat's upsample
  auto bits = [&](uint32_t** p, int lvl, int c) { plan.push_back({(void**)p, (px(lvl) + 1) * words(c) * 4}); };
  for (int k = 0; k < 9; ++k) {
    const int lvl = level_of(k), c = block_of(m, k).conv1.Cout;
    planes(&w.h1[k], lvl, c);
    // res[0]: enc1's general-order conv output ([N][C][H][W]) when it runs
    if (k || D->rgen) planes(&w.res[k], lvl, c);
    bits(&w.a2[k], lvl, c);
    if (k < 4) {
      planes(&w.skip[k], lvl, c);
      bits(&w.skipb[k], lvl, c);
      planes(&w.down[k], lvl + 1, c);
      bits(&w.downb[k], lvl + 1, c);
    } else {
      planes(&w.h2[k], lvl, c);
      if (k < 8) bits(&w.upb[k], lvl, c);
    }
  }
  size_t total = 0;
  for (auto& e : plan) total += (e.second + 255) & ~(size_t)255;
  // another shape that fits the allocation is laid out in it anew (work
  // already enqueued on the same stream finishes first; the tiles of one
  // whole image run on one stream); otherwise a larger one replaces it
  if (!w.base || total > w.cap) {
    if (w.base) { HIP_TRY(hipDeviceSynchronize()); (void)hipFree(w.base); w.base = nullptr; w.cap = 0; }
    HIP_TRY(hipMalloc((void**)&w.base, total));
    w.cap = total;
  }
  size_t off = 0;
  for (auto& e : plan) {
    *e.first = w.base + off;
    off += (e.second + 255) & ~(size_t)255;
  }
  w.N = N; w.H = H; w.W = W;
  return BNN_OK;
}

// work-item shape for the binary conv: the pool epilogue takes 2x2 blocks
// (at most 16 channels), the head one pixel and every channel; otherwise
// the channel group shrinks until the launch has ~4 waves per SIMD
void pick_shape(int epi, int N, int H, int W, int cout, int* mt, int* cog) {
  *mt = epi == EPI_RXPOOL ? 2 : 1;
  if (epi == EPI_RXHEAD) { *cog = cout <= 16 ? 16 : 32; return; }
  const long tiles = (long)N * ((H + *mt - 1) / *mt) * ((W + *mt - 1) / *mt);
  int c = *mt == 2 ? 16 : 32;
  while (c > 8 && c / 2 >= cout) c /= 2;
  auto waves = [&](int g) { return ((tiles + 63) / 64) * (long)((cout + g - 1) / g); };
  while (c > 8 && waves(c) < 4096) c /= 2;
  *cog = c;
}

struct Op {
  const char* label;
  const char* optype;
  double oe, taps;
};

const char* kName[9] = {"enc1", "enc2", "enc3", "enc4", "bott", "dec4", "dec3", "dec2", "dec1"};

int enqueue_forward(const ModelR* m, BnnReactDevice* D, RWorkspace& w, const float* d_in, int N, int H, int W,
                    float* d_logits, hipStream_t s, Dumps* dmp, std::vector<Op>* ops,
                    std::vector<hipEvent_t>* evs, const Scene* sc = nullptr) {
  int hs[5], wsz[5];
  level_dims(H, W, hs, wsz);
  auto mark = [&](const char* label, const char* optype, double oe, double taps) -> int {
    if (!evs) return BNN_OK;
    hipEvent_t e;
    // a timing-only event: no system-scope fence (which would add its own
    // cache writeback to the interval between two kernels)
    HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
    HIP_TRY(hipEventRecord(e, s));
    evs->push_back(e);
    if (label) ops->push_back({label, optype, oe, taps});
    return BNN_OK;
  };
  const bool dump = dmp && dmp->on;
  int pi = 0, rc;
  if ((rc = mark(nullptr, nullptr, 0, 0))) return rc;
  // The forward of patches [nb, nb + cnt) of the batch on stream st.  The
  // float planes are [C][N*h*w] and the bit tensors [N*h*w + 1][words] (a
  // pad pixel after the whole batch), so a part is the same tensors from
  // patch nb on: every pointer moves by nb patches, the planes keep their
  // stride of N patches (ntot), and the pad pixel stays where it is.
  int nb = 0, cnt = N;
  hipStream_t st = s;
  auto pl = [&](const float* p, int lvl) -> float* {
    return p ? const_cast<float*>(p) + (size_t)nb * hs[lvl] * wsz[lvl] : nullptr;
  };
  auto bt = [&](const uint32_t* p, int lvl, int cw) -> uint32_t* {
    return p ? const_cast<uint32_t*>(p) + (size_t)nb * hs[lvl] * wsz[lvl] * cw : nullptr;
  };
  auto part = [&]() -> int {
  {
    const DevBlock& L = D->blk[0];
    RealArgs ra{};
    ra.x = sc ? d_in : d_in + (size_t)nb * D->rcin * H * W;  // a scene part moves prow0 instead
    ra.wm = D->rwm;
    ra.pw = D->rpw;
    ra.alpha = D->ralpha; ra.A = L.e1.A; ra.B = L.e1.B; ra.slope = L.e1.W; ra.rsign = L.t2;
    ra.N = cnt; ra.H = H; ra.W = W; ra.cin = D->rcin; ra.cout = D->rcout;
    ra.out = bt(w.a2[0], 0, words(D->rcout));
    ra.hout = pl(w.h1[0], 0);
    ra.ntot = N;
    ra.f32 = dump ? dmp->conv : nullptr;
    ra.f32b = dump ? dmp->proj : nullptr;
    if (sc) { ra.sH = sc->sH; ra.sW = sc->sW; ra.pcols = sc->pcols; ra.prow0 = sc->prow0 + nb / sc->pcols; }
    if (D->rgen) {
      // the general-order conv, then projection + epilogue + tap
      ra.wm = D->rwm;
      ra.w = D->rw;
      float* conv = dump ? dmp->conv + (size_t)nb * D->rcout * H * W : w.res[0] + (size_t)nb * D->rcout * H * W;
      RealArgs rc1 = ra;
      rc1.out = nullptr;
      rc1.f32 = conv;
      rc1.pw = nullptr;
      rc1.hout = nullptr;
      HIP_TRY(launch_real(rc1, st));
      ReactTailArgs ta{};
      ta.x = ra.x; ta.pw = D->rpw; ta.conv = conv;
      ta.A = L.e1.A; ta.B = L.e1.B; ta.slope = L.e1.W; ta.rsign = L.t2;
      ta.N = cnt; ta.H = H; ta.W = W; ta.cin = D->rcin; ta.cout = D->rcout;
      ta.out = ra.out; ta.hout = ra.hout; ta.ntot = N;
      ta.f32b = dump ? dmp->proj + (size_t)nb * D->rcout * H * W : nullptr;
      ta.sH = ra.sH; ta.sW = ra.sW; ta.pcols = ra.pcols; ta.prow0 = ra.prow0;
      HIP_TRY(launch_react_in_tail(ta, st));
    } else {
      HIP_TRY(launch_react_in(ra, st));
    }
    if ((rc = mark("enc1.u1", "conv_real", (double)N * D->rcout * H * W, (double)D->rcin * 10))) return rc;
  }
  auto proj = [&](int k, const float* x0, int c0, const float* x1, int lvl1, float* out) -> int {
    const DevBlock& L = D->blk[k];
    const int lvl = level_of(k);
    ProjArgs p{};
    p.x0 = pl(x0, lvl); p.x1 = x1 ? pl(x1, lvl1) : nullptr; p.c0 = c0; p.cin = L.cin; p.cout = L.cout;
    p.N = cnt; p.H = hs[lvl]; p.W = wsz[lvl];
    p.ntot = N; p.n0 = nb;
    if (x1) {
      p.h1 = hs[lvl1]; p.w1 = wsz[lvl1];
      const int uH = 2 * p.h1, uW = 2 * p.w1;
      p.oh = p.H > uH ? (p.H - uH) / 2 : 0;
      p.ow = p.W > uW ? (p.W - uW) / 2 : 0;
      p.uh = std::min(uH, p.H);
      p.uw = std::min(uW, p.W);
    }
    p.w = L.pw;
    p.out = pl(out, lvl);
    HIP_TRY(launch_proj(p, st));
    static char lab[9][16];
    snprintf(lab[k], sizeof lab[k], "%s.proj", kName[k]);
    return mark(lab[k], "proj", (double)N * L.cout * p.H * p.W, (double)L.cin);
  };
  // the binary conv of block k (unit u) with a v3 epilogue
  auto bconv = [&](int k, int u, int epi, const uint32_t* in0, const uint32_t* in1, int lvl1, const float* res,
                   const DevEpi& e, const float* trs, float* hout, uint32_t* out, const DevEpi* ed,
                   const float* drs, float* dout, uint32_t* out2) -> int {
    const DevBlock& L = D->blk[k];
    const BlockR& b = block_of(m, k);
    const int lvl = level_of(k);
    BconvArgs a{};
    a.N = cnt; a.H = hs[lvl]; a.W = wsz[lvl];
    a.ntot = N; a.n0 = nb;
    if (u == 1) {
      a.cin = L.cin; a.cout = L.cout; a.cw0 = L.cw0; a.cw1 = L.cw1; a.wt = L.w1; a.pair = L.p1;
    } else {
      a.cin = b.conv2.Cin; a.cout = b.conv2.Cout; a.cw0 = words(a.cin); a.cw1 = 0; a.wt = L.w2; a.pair = L.p2;
    }
    a.in0 = bt(in0, lvl, a.cw0);
    a.in1 = in1 ? bt(in1, lvl1, a.cw1) : nullptr;
    a.padoff = 0x80000000u;
    if (in1) {
      a.h1 = hs[lvl1]; a.w1 = wsz[lvl1];
      const int uH = 2 * a.h1, uW = 2 * a.w1;
      a.oh = a.H > uH ? (a.H - uH) / 2 : 0;
      a.ow = a.W > uW ? (a.W - uW) / 2 : 0;
      a.uh = std::min(uH, a.H);
      a.uw = std::min(uW, a.W);
      a.padoff = (uint32_t)((size_t)(N - nb) * a.h1 * a.w1 * a.cw1 * 4);  // the pad pixel after the batch
    }
    a.cwo = words(a.cout);
    a.res = pl(res, lvl); a.hout = pl(hout, lvl); a.eA = e.A; a.eB = e.B; a.eW = e.W; a.trs = trs;
    a.out = bt(out, lvl, a.cwo);
    if (ed) { a.dA = ed->A; a.dB = ed->B; a.dW = ed->W; }
    a.drs = drs; a.dout = pl(dout, lvl + 1); a.out2 = bt(out2, lvl + 1, a.cwo);
    a.logits = (d_logits && !sc) ? d_logits + (size_t)nb * D->ncls * H * W : d_logits;
    a.hw = D->hw; a.hb = D->hb; a.ncls = D->ncls;
    if (sc && epi == EPI_RXHEAD) {
      a.sH = sc->sH; a.sW = sc->sW; a.pcols = sc->pcols; a.prow0 = sc->prow0 + nb / sc->pcols;
    }
    if (dump) {
      a.P = dmp->P[pi++];
      if (epi == EPI_RXPOOL) a.P2 = dmp->P2[k];
    }
    int mt, cog;
    pick_shape(epi, N, a.H, a.W, a.cout, &mt, &cog);  // the whole batch's shape (parts run side by side)
    HIP_TRY(launch_bconv(a, epi, mt, cog, dump, st));
    static char lab[9][2][16];
    snprintf(lab[k][u - 1], sizeof lab[k][u - 1], "%s.c%d", kName[k], u);
    const char* ot = epi == EPI_RXPOOL ? "bconv_pool" : epi == EPI_RXHEAD ? "bconv_head" : "bconv";
    return mark(lab[k][u - 1], ot, (double)N * a.cout * a.H * a.W, (double)a.cin * 9);
  };
  // encoder: enc1's unit 1 ran above
  for (int k = 0; k < 4; ++k) {
    const DevBlock& L = D->blk[k];
    if (k) {
      if ((rc = proj(k, w.down[k - 1], L.cin, nullptr, 0, w.res[k]))) return rc;
      if ((rc = bconv(k, 1, EPI_RX, w.downb[k - 1], nullptr, 0, w.res[k], L.e1, L.t2, w.h1[k], w.a2[k], nullptr,
                      nullptr, nullptr, nullptr)))
        return rc;
    }
    // skip bits for the decoder that concatenates it, down bits for the next block's tap1
    const float* skip_rs = D->blk[8 - k].t1a;
    const float* down_rs = D->blk[k + 1].t1a;
    if ((rc = bconv(k, 2, EPI_RXPOOL, w.a2[k], nullptr, 0, w.h1[k], L.ea, skip_rs, w.skip[k], w.skipb[k], &L.eb,
                    down_rs, w.down[k], w.downb[k])))
      return rc;
  }
  {
    const DevBlock& L = D->blk[4];
    if ((rc = proj(4, w.down[3], L.cin, nullptr, 0, w.res[4]))) return rc;
    if ((rc = bconv(4, 1, EPI_RX, w.downb[3], nullptr, 0, w.res[4], L.e1, L.t2, w.h1[4], w.a2[4], nullptr, nullptr,
                    nullptr, nullptr)))
      return rc;
    if ((rc = bconv(4, 2, EPI_RX, w.a2[4], nullptr, 0, w.h1[4], L.ea, D->blk[5].t1b, w.h2[4], w.upb[4], nullptr,
                    nullptr, nullptr, nullptr)))
      return rc;
  }
  for (int k = 5; k < 9; ++k) {
    const DevBlock& L = D->blk[k];
    const int lvl = level_of(k), si = 8 - k;
    if ((rc = proj(k, w.skip[si], L.cs, w.h2[k - 1], lvl + 1, w.res[k]))) return rc;
    if ((rc = bconv(k, 1, EPI_RX, w.skipb[si], w.upb[k - 1], lvl + 1, w.res[k], L.e1, L.t2, w.h1[k], w.a2[k],
                    nullptr, nullptr, nullptr, nullptr)))
      return rc;
    if (k < 8) {
      if ((rc = bconv(k, 2, EPI_RX, w.a2[k], nullptr, 0, w.h1[k], L.ea, D->blk[k + 1].t1b, w.h2[k], w.upb[k],
                      nullptr, nullptr, nullptr, nullptr)))
        return rc;
    } else if (block_of(m, k).conv2.Cout <= 32) {
      if ((rc = bconv(k, 2, EPI_RXHEAD, w.a2[k], nullptr, 0, w.h1[k], L.ea, nullptr, dump ? w.h2[k] : nullptr,
                      nullptr, nullptr, nullptr, nullptr, nullptr)))
        return rc;
    } else {
      // a head over more than 32 channels: dec1's h2 planes, then the head
      // on its own (one epilogue group holds at most 32 channels)
      if ((rc = bconv(k, 2, EPI_RX, w.a2[k], nullptr, 0, w.h1[k], L.ea, nullptr, w.h2[k], nullptr, nullptr,
                      nullptr, nullptr, nullptr)))
        return rc;
      HeadArgs h{};
      h.planes = pl(w.h2[k], 0);
      h.plane = (size_t)N * H * W;
      h.cin = block_of(m, k).conv2.Cout;
      h.hw = D->hw; h.hb = D->hb; h.ncls = D->ncls;
      h.N = cnt; h.H = H; h.W = W;
      h.logits = (d_logits && !sc) ? d_logits + (size_t)nb * D->ncls * H * W : d_logits;
      if (sc) { h.sH = sc->sH; h.sW = sc->sW; h.pcols = sc->pcols; h.prow0 = sc->prow0 + nb / sc->pcols; }
      HIP_TRY(launch_head_sep(h, st));
      if ((rc = mark("head", "head", (double)N * D->ncls * H * W, (double)h.cin))) return rc;
    }
  }
  return BNN_OK;
  };
  // A large batch runs as two halves on two streams: the many short
  // kernels of one half fill the launch, ramp and drain gaps of the
  // other's.  A scene splits at whole patch rows; one stream with
  // per-kernel events or debug dumps.
  const int unit = sc ? sc->pcols : 1;
  const bool split = !dump && !evs && N >= 256 && N / unit >= 2;
  if (!split) return part();
  if (!D->side) {
    // all or nothing: a failure leaves no half-made set behind
    hipStream_t side = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    if (hipStreamCreateWithFlags(&side, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&join, hipEventDisableTiming) != hipSuccess) {
      if (join) (void)hipEventDestroy(join);
      if (fork) (void)hipEventDestroy(fork);
      if (side) (void)hipStreamDestroy(side);
      return set_err(BNN_EHIP, "cannot create the stream of a split batch");
    }
    D->side = side; D->ev_fork = fork; D->ev_join = join;
  }
  HIP_TRY(hipEventRecord(D->ev_fork, s));
  HIP_TRY(hipStreamWaitEvent(D->side, D->ev_fork, 0));
  const int half = (N / unit) / 2 * unit;
  nb = 0; cnt = half; st = s;
  if ((rc = part())) return rc;
  nb = half; cnt = N - half; st = D->side;
  if ((rc = part())) return rc;
  HIP_TRY(hipEventRecord(D->ev_join, D->side));
  HIP_TRY(hipStreamWaitEvent(s, D->ev_join, 0));
  return BNN_OK;
}

// A launch addresses its input with 32-bit byte offsets, so one launch
// takes less than 2 GiB of it: a batch runs in sub-batches of that size
// (patches_per_launch), a cube of 2 GiB or more in strips of whole patch
// rows (run_patched_strips), one image of 2 GiB or more in tiles
// (run_tiles).
constexpr size_t kLaunchBytes = 0x7FFFFFF0ull;
int patches_per_launch(const ModelR* m, int H, int W) {
  return (int)std::min<size_t>(1 << 30, (kLaunchBytes - 1) / ((size_t)m->n_bands * H * W * 4));
}

int check_shape(const ModelR* m, int N, int H, int W) {
  if (!m || !m->dev) return set_err(BNN_EARG, "model not loaded");
  if (N < 0) return set_err(BNN_EARG, "negative batch");
  if (H < 16 || W < 16) return set_err(BNN_EARG, "H=%d W=%d: the four 2x2 pools need H, W >= 16", H, W);
  return BNN_OK;
}

int run_device_launch(const ModelR* m, const float* d_in, int N, int H, int W, float* d_logits, hipStream_t s,
                      Dumps* dmp, const Scene* sc);
int grow(float** p, size_t* cap, size_t bytes);

// An image whose input passes the per-launch limit (or, for tests, the tile
// budget BNN_TILE_BYTES) runs in tiles exactly as the v1 forward's whole
// images do (bnn_host.cpp, kTileHalo): full-width row strips, or square
// tiles, with core edges on multiples of 16 px and 128 px of the image
// around each core.  The v3 chain has the same contamination depth from a
// tile's inner edge: two 3x3 binary convs per block at each level (its 1x1
// projections and epilogues stay on their pixel), 2x2 pools and nearest
// upsamples between levels, so 94 px.
constexpr int kTileHalo = 128;

size_t tile_budget() {
  const char* e = getenv("BNN_TILE_BYTES");
  const size_t def = (size_t)1 << 30;
  if (!e || !*e) return def;
  const long long v = atoll(e);
  return v >= (1 << 20) ? (size_t)v : def;
}

bool needs_tiles(const ModelR* m, int H, int W) {
  return patches_per_launch(m, H, W) < 1 || (size_t)m->n_bands * H * W * 4 > tile_budget();
}

int plan_tiles(const ModelR* m, int H, int W, int* th, int* tw) {
  const size_t px = (size_t)m->n_bands * 4, bud = std::min(tile_budget(), kLaunchBytes - 1);
  const size_t rows = bud / (px * W);
  if (rows >= (size_t)2 * kTileHalo + 16) {
    *tw = W;
    *th = (int)std::min<size_t>((rows - 2 * kTileHalo) / 16 * 16, (size_t)H);
    return BNN_OK;
  }
  size_t side = 16;
  while ((side + 16) * (side + 16) * px <= bud) side += 16;
  if (side < (size_t)2 * kTileHalo + 16)
    return set_err(BNN_EARG, "%d bands: a tile of %d px (16 + 2 x %d halo) exceeds the tile budget", m->n_bands,
                   16 + 2 * kTileHalo, kTileHalo);
  *th = *tw = (int)(side - 2 * kTileHalo);
  return BNN_OK;
}

// The tiles of N whole images (host or device pointers) through the strip
// staging buffers (a streamed file's cube sits in stage_in), in order on s.
int run_tiles(const ModelR* m, const float* in, bool in_host, int N, int H, int W, float* out, bool out_host,
              hipStream_t s) {
  int rc, th, tw;
  if ((rc = plan_tiles(m, H, W, &th, &tw))) return rc;
  BnnReactDevice* D = m->dev;
  const int nb = m->n_bands, nc = m->n_classes;
  const int fh = std::min(H, th + 2 * kTileHalo), fw = std::min(W, tw + 2 * kTileHalo);
  if ((rc = grow(&D->strip_in, &D->strip_in_cap, (size_t)nb * fh * fw * 4))) return rc;
  if ((rc = grow(&D->strip_out, &D->strip_out_cap, (size_t)nc * fh * fw * 4))) return rc;
  const hipMemcpyKind kin = in_host ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice;
  const hipMemcpyKind kout = out_host ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice;
  for (int n = 0; n < N; ++n) {
    const float* img = in + (size_t)n * nb * H * W;
    float* lg = out + (size_t)n * nc * H * W;
    for (int r0 = 0; r0 < H; r0 += th)
      for (int c0 = 0; c0 < W; c0 += tw) {
        const int r1 = std::min(H, r0 + th), c1 = std::min(W, c0 + tw);
        const int a0 = std::max(0, r0 - kTileHalo), a1 = std::min(H, r1 + kTileHalo);
        const int b0 = std::max(0, c0 - kTileHalo), b1 = std::min(W, c1 + kTileHalo);
        const int h = a1 - a0, w = b1 - b0;
        if (h < 16 || w < 16) return set_err(BNN_EARG, "tile %dx%d at (%d, %d): below 16 px", h, w, a0, b0);
        if (w == W) {
          HIP_TRY(hipMemcpy2DAsync(D->strip_in, (size_t)h * W * 4, img + (size_t)a0 * W, (size_t)H * W * 4,
                                   (size_t)h * W * 4, nb, kin, s));
        } else {
          for (int c = 0; c < nb; ++c)
            HIP_TRY(hipMemcpy2DAsync(D->strip_in + (size_t)c * h * w, (size_t)w * 4,
                                     img + (size_t)c * H * W + (size_t)a0 * W + b0, (size_t)W * 4, (size_t)w * 4, h,
                                     kin, s));
        }
        if ((rc = run_device_launch(m, D->strip_in, 1, h, w, D->strip_out, s, nullptr, nullptr))) return rc;
        for (int c = 0; c < nc; ++c)
          HIP_TRY(hipMemcpy2DAsync(lg + (size_t)c * H * W + (size_t)r0 * W + c0, (size_t)W * 4,
                                   D->strip_out + (size_t)c * h * w + (size_t)(r0 - a0) * w + (c0 - b0),
                                   (size_t)w * 4, (size_t)(c1 - c0) * 4, r1 - r0, kout, s));
      }
  }
  return BNN_OK;
}

// One launch's forward (N below patches_per_launch).
int run_device_launch(const ModelR* m, const float* d_in, int N, int H, int W, float* d_logits, hipStream_t s,
                      Dumps* dmp, const Scene* sc) {
  int rc;
  BnnReactDevice* D = m->dev;
  if ((rc = ensure_ws(m, D, D->ws, N, H, W))) return rc;
  if (!prof_enabled()) return enqueue_forward(m, D, D->ws, d_in, N, H, W, d_logits, s, dmp, nullptr, nullptr, sc);
  std::vector<Op> ops;
  std::vector<hipEvent_t> evs;
  rc = enqueue_forward(m, D, D->ws, d_in, N, H, W, d_logits, s, dmp, &ops, &evs, sc);
  if (!rc && !evs.empty()) {
    HIP_TRY(hipEventSynchronize(evs.back()));
    for (size_t i = 0; i + 1 < evs.size() && i < ops.size(); ++i) {
      float ms = 0;
      HIP_TRY(hipEventElapsedTime(&ms, evs[i], evs[i + 1]));
      prof_add(ops[i].label, ops[i].optype, ops[i].oe, ops[i].taps, ms * 1e-3);
    }
  }
  for (hipEvent_t e : evs) (void)hipEventDestroy(e);
  return rc;
}

// A batch in sub-batches of one launch each (the debug forward's dumps
// cover the whole batch and take one launch).
int run_device(const ModelR* m, const float* d_in, int N, int H, int W, float* d_logits, hipStream_t s,
               Dumps* dmp, const Scene* sc = nullptr) {
  int rc;
  if ((rc = check_shape(m, N, H, W))) return rc;
  if (N == 0) return BNN_OK;
  if (!sc && needs_tiles(m, H, W)) {
    if (dmp && dmp->on) return set_err(BNN_EARG, "a debug forward takes images of at most 2 GiB");
    return run_tiles(m, d_in, false, N, H, W, d_logits, false, s);
  }
  const int per = patches_per_launch(m, H, W);
  if ((dmp && dmp->on) || sc || N <= per) return run_device_launch(m, d_in, N, H, W, d_logits, s, dmp, sc);
  for (int n0 = 0; n0 < N; n0 += per) {
    const int cnt = std::min(per, N - n0);
    if ((rc = run_device_launch(m, d_in + (size_t)n0 * m->n_bands * H * W, cnt, H, W,
                                d_logits + (size_t)n0 * m->n_classes * H * W, s, nullptr, nullptr)))
      return rc;
  }
  return BNN_OK;
}

int grow(float** p, size_t* cap, size_t bytes) {
  if (*cap >= bytes) return BNN_OK;
  if (*p) { HIP_TRY(hipDeviceSynchronize()); (void)hipFree(*p); *p = nullptr; *cap = 0; }
  HIP_TRY(hipMalloc((void**)p, bytes ? bytes : 4));
  *cap = bytes;
  return BNN_OK;
}

// Host input -> host logits, in sub-batches of at most one launch each
// (staging buffers of one sub-batch, so device memory stays bounded).
int run_host(const ModelR* m, const float* input, int N, int H, int W, float* logits, Dumps* dmp) {
  int rc;
  if ((rc = check_shape(m, N, H, W))) return rc;
  if (N == 0) return BNN_OK;
  BnnReactDevice* D = m->dev;
  const bool dump = dmp && dmp->on;
  if (needs_tiles(m, H, W)) {
    if (dump) return set_err(BNN_EARG, "a debug forward takes images of at most 2 GiB");
    if ((rc = run_tiles(m, input, true, N, H, W, logits, true, D->stream))) return rc;
    HIP_TRY(hipStreamSynchronize(D->stream));
    return BNN_OK;
  }
  const int per = dump ? N : std::min(N, patches_per_launch(m, H, W));
  const size_t pin = (size_t)m->n_bands * H * W, pout = (size_t)m->n_classes * H * W;
  if ((rc = grow(&D->stage_in, &D->stage_in_cap, per * pin * 4))) return rc;
  if ((rc = grow(&D->stage_out, &D->stage_out_cap, per * pout * 4))) return rc;
  for (int n0 = 0; n0 < N; n0 += per) {
    const int cnt = std::min(per, N - n0);
    HIP_TRY(hipMemcpyAsync(D->stage_in, input + (size_t)n0 * pin, cnt * pin * 4, hipMemcpyHostToDevice,
                           D->stream));
    if ((rc = run_device_launch(m, D->stage_in, cnt, H, W, D->stage_out, D->stream, dmp, nullptr))) return rc;
    HIP_TRY(hipMemcpyAsync(logits + (size_t)n0 * pout, D->stage_out, cnt * pout * 4, hipMemcpyDeviceToHost,
                           D->stream));
    HIP_TRY(hipStreamSynchronize(D->stream));
  }
  return BNN_OK;
}

// Patch-wise forward with the tiling of csrc/bnn_model_react.c:454-476: P x P
// patches at multiples of P, an edge patch zero past the image, every patch
// its own image, its logits inside the image stitched into the map.  The
// enc1 kernel reads the patches straight out of the cube and the head
// writes the map (scene mode), in launches of whole patch rows.
int check_patched(const ModelR* m, int H, int W, int P) {
  if (!m || !m->dev) return set_err(BNN_EARG, "model not loaded");
  if (P < 16 || P % 16) return set_err(BNN_EARG, "patch size %d must be a positive multiple of 16", P);
  if (H <= 0 || W <= 0) return set_err(BNN_EARG, "bad image size %dx%d", H, W);
  // one row of patches must fit a launch (strips are whole patch rows)
  if ((size_t)m->n_bands * P * W * 4 >= kLaunchBytes)
    return set_err(BNN_EARG, "one row of %dx%d patches of a %d-wide image exceeds a launch (2 GiB)", P, P, W);
  return BNN_OK;
}

// a cube the kernels can address in place (32-bit byte offsets)
bool cube_in_place(const ModelR* m, int H, int W) { return (size_t)m->n_bands * H * W * 4 < kLaunchBytes; }

int run_patched_rows(const ModelR* m, const float* d_cube, int H, int W, float* d_map, int P, hipStream_t s) {
  const int prows = (H + P - 1) / P, pcols = (W + P - 1) / P;
  // about 1024 patches per launch
  const int rows_per = std::max(1, 1024 / pcols);
  for (int r0 = 0; r0 < prows; r0 += rows_per) {
    const int nr = std::min(rows_per, prows - r0);
    const Scene sc{H, W, pcols, r0};
    int rc;
    if ((rc = run_device(m, d_cube, nr * pcols, P, P, d_map, s, nullptr, &sc))) return rc;
  }
  return BNN_OK;
}

// A cube of 2 GiB or more, by strips: R whole patch rows (R*P image rows,
// fewer at the bottom edge) at a time, copied into a sub-cube [nb][rows][W]
// and run as an image of `rows` rows; its map rows [ncls][rows][W] go to the
// full map, one contiguous run per class since a strip spans the width.
// Every launch then addresses at most one strip.  A host cube is copied
// band by band (each band's strip rows are contiguous).
int run_patched_strips(const ModelR* m, const float* cube, bool host_cube, int H, int W, float* map, bool host_map,
                       int P, hipStream_t s) {
  BnnReactDevice* D = m->dev;
  const int nb = m->n_bands, ncls = m->n_classes;
  const int prows = (H + P - 1) / P;
  const size_t row_bytes = (size_t)nb * P * W * 4;
  // strips of about 256 MB of input
  const int R = std::max(1, (int)std::min<size_t>(prows, (256u << 20) / row_bytes));
  int rc;
  if ((rc = grow(&D->strip_in, &D->strip_in_cap, row_bytes * R))) return rc;
  if ((rc = grow(&D->strip_out, &D->strip_out_cap, (size_t)ncls * R * P * W * 4))) return rc;
  for (int pr0 = 0; pr0 < prows; pr0 += R) {
    const int nr = std::min(R, prows - pr0);
    const int r0 = pr0 * P, rows = std::min(nr * P, H - r0);
    const size_t band = (size_t)rows * W;
    if (host_cube) {
      for (int b = 0; b < nb; ++b)
        HIP_TRY(hipMemcpyAsync(D->strip_in + b * band, cube + ((size_t)b * H + r0) * W, band * 4,
                               hipMemcpyHostToDevice, s));
    } else {
      HIP_TRY(hipMemcpy2DAsync(D->strip_in, band * 4, cube + (size_t)r0 * W, (size_t)H * W * 4, band * 4, nb,
                               hipMemcpyDeviceToDevice, s));
    }
    if ((rc = run_patched_rows(m, D->strip_in, rows, W, D->strip_out, P, s))) return rc;
    for (int c = 0; c < ncls; ++c)
      HIP_TRY(hipMemcpyAsync(map + ((size_t)c * H + r0) * W, D->strip_out + c * band, band * 4,
                             host_map ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice, s));
    if (host_map) HIP_TRY(hipStreamSynchronize(s));
  }
  return BNN_OK;
}

int run_patched_device(const ModelR* m, const float* d_cube, int H, int W, float* d_map, int P, hipStream_t s) {
  int rc;
  if ((rc = check_patched(m, H, W, P))) return rc;
  if (cube_in_place(m, H, W)) return run_patched_rows(m, d_cube, H, W, d_map, P, s);
  return run_patched_strips(m, d_cube, false, H, W, d_map, false, P, s);
}

int run_patched_host(const ModelR* m, const float* cube, int H, int W, float* map, int P) {
  int rc;
  if ((rc = check_patched(m, H, W, P))) return rc;
  BnnReactDevice* D = m->dev;
  if (!cube_in_place(m, H, W)) return run_patched_strips(m, cube, true, H, W, map, true, P, D->stream);
  const size_t nin = (size_t)m->n_bands * H * W, nout = (size_t)m->n_classes * H * W;
  if ((rc = grow(&D->stage_in, &D->stage_in_cap, nin * 4))) return rc;
  if ((rc = grow(&D->stage_out, &D->stage_out_cap, nout * 4))) return rc;
  HIP_TRY(hipMemcpyAsync(D->stage_in, cube, nin * 4, hipMemcpyHostToDevice, D->stream));
  if ((rc = run_patched_rows(m, D->stage_in, H, W, D->stage_out, P, D->stream))) return rc;
  HIP_TRY(hipMemcpyAsync(map, D->stage_out, nout * 4, hipMemcpyDeviceToHost, D->stream));
  HIP_TRY(hipStreamSynchronize(D->stream));
  return BNN_OK;
}

// Row strips of a streamed input file hold this many floats (4 MiB).
constexpr size_t kStripFloats = size_t(1) << 20;

// The [nb,H,W] float32 cube in f, from the start of the file, into
// D->stage_in, as the reference's file reader takes it: band by band, rows
// r0..r1 of a band at their absolute offset (csrc/bnn_model_react.c:505-520).
// Each strip of whole rows goes through one of two pinned buffers and is
// copied on D->stream while the next one is read, so host memory never holds
// the cube.  A short read fails with the reference's message.
int stream_cube(BnnReactDevice* D, FILE* f, int nb, int H, int W) {
  if (!f) return set_err(BNN_EARG, "null input file");
  const size_t plane = (size_t)H * W;
  int rc;
  if ((rc = grow(&D->stage_in, &D->stage_in_cap, (size_t)nb * plane * 4))) return rc;
  for (int k = 0; k < 2; ++k) {
    if (!D->strip[k]) HIP_TRY(hipHostMalloc((void**)&D->strip[k], kStripFloats * 4, hipHostMallocDefault));
    if (!D->strip_done[k]) HIP_TRY(hipEventCreateWithFlags(&D->strip_done[k], hipEventDisableTiming));
  }
  int rows = (int)std::min<size_t>(H, kStripFloats / (size_t)W);
  // BNN_STREAM_ROWS=<r> caps a strip at r rows (any r >= 1 gives the same
  // cube; tests use it to cross many strip boundaries on small images)
  if (const char* e = getenv("BNN_STREAM_ROWS")) rows = std::min(rows, std::max(1, atoi(e)));
  if (rows < 1) return set_err(BNN_EARG, "image rows of %d floats exceed a %zu-float strip", W, kStripFloats);
  bool used[2] = {false, false};
  int k = 0;
  for (int b = 0; b < nb; ++b) {
    for (int r0 = 0; r0 < H; r0 += rows, k ^= 1) {
      const int r1 = std::min(H, r0 + rows);
      const size_t n = (size_t)(r1 - r0) * W;
      if (used[k]) HIP_TRY(hipEventSynchronize(D->strip_done[k]));  // its last copy has left
      const off_t at = (off_t)(((size_t)b * H + r0) * W * 4);
      if (fseeko(f, at, SEEK_SET) != 0 || fread(D->strip[k], 4, n, f) != n)
        return set_err(BNN_EARG, "file_reader: short read band %d rows %d..%d", b, r0, r1);
      HIP_TRY(hipMemcpyAsync(D->stage_in + b * plane + (size_t)r0 * W, D->strip[k], n * 4, hipMemcpyHostToDevice,
                             D->stream));
      HIP_TRY(hipEventRecord(D->strip_done[k], D->stream));
      used[k] = true;
    }
  }
  return BNN_OK;
}

// The forward of a streamed file: whole image (P = 0) or patch-wise.
int run_file(const ModelR* m, FILE* f, int H, int W, float* logits, int P) {
  if (!m || !m->dev) return set_err(BNN_EARG, "model not loaded");
  int rc;
  if (!P && (rc = check_shape(m, 1, H, W))) return rc;
  if (P && (rc = check_patched(m, H, W, P))) return rc;
  BnnReactDevice* D = m->dev;
  const size_t nout = (size_t)m->n_classes * H * W;
  if ((rc = stream_cube(D, f, m->n_bands, H, W))) return rc;
  if ((rc = grow(&D->stage_out, &D->stage_out_cap, nout * 4))) return rc;
  rc = P ? run_patched_device(m, D->stage_in, H, W, D->stage_out, P, D->stream)
         : run_device(m, D->stage_in, 1, H, W, D->stage_out, D->stream, nullptr);
  if (rc) return rc;
  HIP_TRY(hipMemcpyAsync(logits, D->stage_out, nout * 4, hipMemcpyDeviceToHost, D->stream));
  HIP_TRY(hipStreamSynchronize(D->stream));
  return BNN_OK;
}

// ------------------------------------------------------------ debug forward
// planes [C][N*HW] -> [N][C][HW]
std::vector<float> planes_to_nchw(const float* d, int N, int C, int HW) {
  std::vector<float> p((size_t)C * N * HW), out(p.size());
  if (hipMemcpy(p.data(), d, p.size() * 4, hipMemcpyDeviceToHost) != hipSuccess) return {};
  for (int c = 0; c < C; ++c)
    for (int n = 0; n < N; ++n)
      memcpy(&out[((size_t)n * C + c) * HW], &p[((size_t)c * N + n) * HW], (size_t)HW * 4);
  return out;
}
// bits [N][HW][cw] (+ pad pixel) -> int8 +-1 [N][C][HW]
std::vector<int8_t> bits_to_nchw(const uint32_t* d, int N, int C, int HW) {
  const int cw = words(C);
  std::vector<uint32_t> b((size_t)N * HW * cw);
  std::vector<int8_t> out((size_t)N * C * HW);
  if (hipMemcpy(b.data(), d, b.size() * 4, hipMemcpyDeviceToHost) != hipSuccess) return {};
  for (int n = 0; n < N; ++n)
    for (int p = 0; p < HW; ++p)
      for (int c = 0; c < C; ++c)
        out[((size_t)n * C + c) * HW + p] = ((b[((size_t)n * HW + p) * cw + (c >> 5)] >> (c & 31)) & 1u) ? 1 : -1;
  return out;
}

}  // namespace

// ----------------------------------------------------------------- C ABI
extern "C" {

int bnn_react_blob_check(const char* path) {
  ModelR* m = nullptr;
  int rc = parse_blob(path, &m);
  if (rc) return rc;
  rc = validate(m);
  free_host(m);
  return rc;
}

void bnn_free_react(ModelR* m) {
  if (!m) return;
  if (m->dev) {
    release(m->dev);
    delete m->dev;
    m->dev = nullptr;
  }
  free_host(m);
}

int bnn_react_load_status(const char* path, ModelR** out) {
  if (!out) return set_err(BNN_EARG, "null output pointer");
  *out = nullptr;
  ModelR* m = nullptr;
  int rc = parse_blob(path, &m);
  if (rc) return rc;
  if ((rc = validate(m)) || (rc = build_device(m))) {
    bnn_free_react(m);
    return rc;
  }
  *out = m;
  return BNN_OK;
}

ModelR* bnn_load_react(const char* path) {
  ModelR* m = nullptr;
  if (bnn_react_load_status(path, &m)) die();
  return m;
}

int bnn_react_forward_batch(const ModelR* m, const float* input, int N, int H, int W, float* logits) {
  return run_host(m, input, N, H, W, logits, nullptr);
}

void bnn_forward_react(const ModelR* m, const float* input, int H, int W, float* logits) {
  if (run_host(m, input, 1, H, W, logits, nullptr)) die();
}

int bnn_react_forward_device(const ModelR* m, const float* d_input, int N, int H, int W, float* d_logits,
                             void* stream) {
  if (!m || !m->dev) return set_err(BNN_EARG, "model not loaded");
  // NULL is the HIP default stream, as for every stream argument in HIP
  return run_device(m, d_input, N, H, W, d_logits, (hipStream_t)stream, nullptr);
}

void* bnn_react_stream(const ModelR* m) { return (m && m->dev) ? (void*)m->dev->stream : nullptr; }

void bnn_forward_react_file(const ModelR* m, FILE* in_f, int H, int W, float* logits) {
  if (run_file(m, in_f, H, W, logits, 0)) die();
}

void bnn_forward_react_patched(const ModelR* m, const float* input, int H, int W, float* logits, int P) {
  if (run_patched_host(m, input, H, W, logits, P)) die();
}

int bnn_react_forward_patched(const ModelR* m, const float* input, int H, int W, float* logits, int P) {
  return run_patched_host(m, input, H, W, logits, P);
}

void bnn_forward_react_patched_file(const ModelR* m, FILE* f, int H, int W, float* logits, int P) {
  if (run_file(m, f, H, W, logits, P)) die();
}

int bnn_react_forward_patched_device(const ModelR* m, const float* d_input, int H, int W, float* d_logits, int P,
                                     void* stream) {
  if (!m || !m->dev) return set_err(BNN_EARG, "model not loaded");
  return run_patched_device(m, d_input, H, W, d_logits, P, (hipStream_t)stream);
}

int bnn_react_forward_debug(const ModelR* m, const float* input, int N, int H, int W, float* logits,
                            bnn_react_stage_cb cb, void* ctx) {
  int rc;
  if ((rc = check_shape(m, N, H, W))) return rc;
  if (N == 0) return BNN_OK;
  BnnReactDevice* D = m->dev;
  int hs[5], wsz[5];
  level_dims(H, W, hs, wsz);
  // P dumps: conv1 (not enc1) and conv2 of every block, in launch order
  std::vector<void*> bufs;
  bool oom = false;  // any failed allocation: no dump kernel may run with a null target
  auto alloc = [&](size_t bytes) -> void* {
    void* p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 4) != hipSuccess) {
      (void)hipGetLastError();
      oom = true;
      return nullptr;
    }
    bufs.push_back(p);
    return p;
  };
  Dumps dm;
  dm.on = true;
  const int C1 = m->enc[0].conv1.Cout;
  dm.conv = (float*)alloc((size_t)N * C1 * H * W * 4);
  dm.proj = (float*)alloc((size_t)N * C1 * H * W * 4);
  struct PInfo { int k, u, lvl, c; };
  std::vector<PInfo> pinfo;
  for (int k = 0; k < 9; ++k) {
    const BlockR& b = block_of(m, k);
    if (k) pinfo.push_back({k, 1, level_of(k), b.conv1.Cout});
    pinfo.push_back({k, 2, level_of(k), b.conv2.Cout});
    if (k < 4) dm.P2[k] = (int32_t*)alloc((size_t)N * b.conv2.Cout * hs[k + 1] * wsz[k + 1] * 4);
  }
  for (size_t i = 0; i < pinfo.size(); ++i)
    dm.P[i] = (int32_t*)alloc((size_t)N * pinfo[i].c * hs[pinfo[i].lvl] * wsz[pinfo[i].lvl] * 4);
  if (oom) {
    for (void* q : bufs) (void)hipFree(q);
    return set_err(BNN_EHIP, "out of device memory for the debug dumps (N=%d)", N);
  }
  rc = run_host(m, input, N, H, W, logits, &dm);
  if (!rc && cb) {
    RWorkspace& w = D->ws;
    auto emitf = [&](const char* name, const std::vector<float>& v, int C, int h, int wd) {
      cb(ctx, name, 2, N, C, h, wd, v.data());
    };
    auto emitb = [&](const char* name, const std::vector<int8_t>& v, int C, int h, int wd) {
      cb(ctx, name, 0, N, C, h, wd, v.data());
    };
    auto emitP = [&](const char* name, const int32_t* d, int C, int h, int wd) {
      std::vector<int32_t> v((size_t)N * C * h * wd);
      if (hipMemcpy(v.data(), d, v.size() * 4, hipMemcpyDeviceToHost) == hipSuccess) cb(ctx, name, 1, N, C, h, wd, v.data());
    };
    char nm[48];
    {
      std::vector<float> v((size_t)N * C1 * H * W);
      if (hipMemcpy(v.data(), dm.proj, v.size() * 4, hipMemcpyDeviceToHost) == hipSuccess) emitf("enc1.u1.proj", v, C1, H, W);
      if (hipMemcpy(v.data(), dm.conv, v.size() * 4, hipMemcpyDeviceToHost) == hipSuccess) emitf("enc1.u1.conv", v, C1, H, W);
    }
    size_t pi = 0;
    for (int k = 0; k < 9; ++k) {
      const BlockR& b = block_of(m, k);
      const int lvl = level_of(k), h = hs[lvl], wd = wsz[lvl], HW = h * wd, c = b.conv1.Cout;
      if (k) {
        snprintf(nm, sizeof nm, "%s.u1.proj", kName[k]);
        emitf(nm, planes_to_nchw(w.res[k], N, c, HW), c, h, wd);
        if (k <= 4) {  // the tap1 bits are the previous block's down bits
          snprintf(nm, sizeof nm, "%s.u1.tap", kName[k]);
          emitb(nm, bits_to_nchw(w.downb[k - 1], N, b.conv1.Cin, HW), b.conv1.Cin, h, wd);
        }
        snprintf(nm, sizeof nm, "%s.u1.P", kName[k]);
        emitP(nm, dm.P[pi++], c, h, wd);
      }
      snprintf(nm, sizeof nm, "%s.h1", kName[k]);
      emitf(nm, planes_to_nchw(w.h1[k], N, c, HW), c, h, wd);
      snprintf(nm, sizeof nm, "%s.u2.tap", kName[k]);
      emitb(nm, bits_to_nchw(w.a2[k], N, c, HW), c, h, wd);
      snprintf(nm, sizeof nm, "%s.u2.P", kName[k]);
      emitP(nm, dm.P[pi++], c, h, wd);
      if (k < 4) {
        const int h2 = hs[lvl + 1], w2 = wsz[lvl + 1];
        snprintf(nm, sizeof nm, "%s.skip", kName[k]);
        emitf(nm, planes_to_nchw(w.skip[k], N, c, HW), c, h, wd);
        snprintf(nm, sizeof nm, "%s.pool.P", kName[k]);
        emitP(nm, dm.P2[k], c, h2, w2);
        snprintf(nm, sizeof nm, "%s.down", kName[k]);
        emitf(nm, planes_to_nchw(w.down[k], N, c, h2 * w2), c, h2, w2);
      } else {
        snprintf(nm, sizeof nm, "%s.h2", kName[k]);
        emitf(nm, planes_to_nchw(w.h2[k], N, c, HW), c, h, wd);
      }
    }
    std::vector<float> lg(logits, logits + (size_t)N * m->n_classes * H * W);
    cb(ctx, "logits", 2, N, m->n_classes, H, W, lg.data());
  }
  for (void* p : bufs) (void)hipFree(p);
  return rc;
}

}  // extern "C"
