// bnn_kernels.h - device-side argument blocks and launchers (internal).
//
// HBM layouts used by every kernel here:
//   real input      float  [N][Cin][H][W]       (per patch [band,row,col], csrc/main.c:3)
//   binary act      uint32 [N][H][W][CW]        bit (c & 31) of word (c >> 5) = (a_c > 0),
//                                               CW = ceil(C/32); unused high bits are 0
//   binary weights  uint32 [CW][Cout][9]        same channel->bit map as the activations
//                                               they meet, per 3x3 tap t = ky*3+kx
//   real weights    float  [ceil(Cout/G)][Cin][9][G] +-1.0 (groups of G =
//                                               kRealGroup output channels, zero-padded), t = ky*3+kx
//   logits          float  [N][ncls][H][W]
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

namespace bnn {

enum Epi : int {
  EPI_FOLD = 0,  // integer rule on P -> packed bits
  EPI_POOL = 1,  // rule on P (skip) + 2x2 max of P -> second rule (down)
  EPI_HEAD = 2,  // rule on P -> +-1 -> fp32 1x1 head -> logits
  EPI_P = 3,     // raw int32 P [N][Cout][H][W]
  // v3 (ReActNet real highway): h = RPReLU(A*P + (B + move1) + res) as
  // float planes, and the bits of the next tap on h
  EPI_RX = 4,      // h and its tap bits
  EPI_RXPOOL = 5,  // skip h (+ bits) and the pooled down h (+ bits)
  EPI_RXHEAD = 6,  // h, then the fp32 1x1 head -> logits
};

// One modular interval per channel: bit = (uint32)(P - lo) < wid.  Covers
// every integer rule type (csrc/bnn_fold.c:37-60); a complemented interval
// [lo, lo+wid) is the interval [lo+wid, lo+2^32), so no inversion flag is
// needed.  Arrays are padded to a multiple of 32 channels with wid = 0.
struct FoldDev {
  const int32_t* lo;
  const uint32_t* wid;
};

// n / d by multiply-high for 0 <= n < 2^31: q = d == 1 ? n : mulhi(n, mul) >> shr
// with mul = ceil(2^p / d), p = 31 + ceil(log2 d), shr = p - 32.
struct FastDiv {
  uint32_t d, mul, shr;
};
inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f{d, 0u, 0u};
  if (d <= 1) return f;
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  const uint32_t p = 31 + l;
  f.mul = (uint32_t)(((1ull << p) + d - 1) / d);
  f.shr = p - 32;
  return f;
}

struct BconvArgs {
  const uint32_t* in0;  // plain input, or the skip half of a concat
  const uint32_t* in1;  // low-res tensor upsampled 2x nearest (concat), or null
  int cw0, cw1;         // words per pixel of in0 / in1
  int h1, w1;           // in1 spatial dims
  int oh, ow;           // F.pad before-offsets of the upsample inside H x W
  int uh, uw;           // rows/cols of H x W the upsample covers (from oh/ow)
  int N, H, W;
  int cin, cout;        // true channel counts
  uint32_t ntiles;      // N * tiles per patch (set by launch_bconv)
  int xorder;           // XCD-aware block order (set by launch_bconv)
  FastDiv dper, dtw;    // tiles per patch, tiles per row (set by launch_bconv)
  const uint32_t* wt;   // [cw0+cw1][cout][9], or (pair) [cout][5] then [cw1][cout][9]
  // a first segment (plain input, or a concat's skip part) of at most 16
  // channels: two taps share a 32-bit word, tap 2p in the low half, 2p+1 in
  // the high half (tap 8 alone), so 5 popcounts per output channel there
  // instead of 9
  int pair;
  FoldDev f1, f2;
  uint32_t* out;        // bits [N][H][W][cwo]  (EPI_FOLD/POOL)
  uint32_t* out2;       // pooled bits [N][H/2][W/2][cwo] (EPI_POOL)
  int cwo;
  int32_t* P;           // EPI_P output, or the P dump of a fused epilogue
  int32_t* P2;          // pooled-P dump (EPI_POOL)
  float* logits;        // EPI_HEAD: [N][ncls][H][W], or the scene map [ncls][sH][sW]
  const float* hw;      // head W [ncls][cout]
  const float* hb;      // head bias [ncls]
  int ncls;
  int sH, sW, pcols, prow0;  // scene mode (pcols > 0), as in RealArgs
  // in1 byte offset read where the upsample does not cover an in-image
  // position: 0x80000000 (past the buffer: reads 0 bits, v1's zero-filled
  // concat) or the offset of the pad pixel that holds the tap bits of 0.0
  // (v3's zero-filled float concat)
  uint32_t padoff;
  // v3 epilogues.  Float planes: element (c, n, y, x) at c*N*H*W + (n*H + y)*W + x.
  const float* res;     // shortcut planes [cout] at this resolution
  float* hout;          // h planes (EPI_RXHEAD: optional)
  const float *eA, *eB, *eW;   // A, B + move1, PReLU weight; padded to 32
  const float* trs;     // rsign of the tap on h -> out bits (+ the pad pixel at N*H*W), or null
  const float *dA, *dB, *dW, *drs;  // EPI_RXPOOL: the pooled-down epilogue and its tap -> out2
  float* dout;          // EPI_RXPOOL: pooled h planes at (H/2, W/2)
  // v3 batch parts: the planes and bit tensors hold ntot patches and this
  // call covers N of them from patch n0, its pointers already moved to n0
  // (ntot 0: the call covers the whole batch)
  int ntot, n0;
};

struct RealArgs {
  const float* x;
  const float* w;       // [ceil(cout/G)][cin][9][G] (vector-ALU kernel)
  const uint64_t* wm;   // [ceil(cout/16)][cin padded][3] lane masks (matrix-core kernel), or null
  // certified fp16 matrix-core kernel (launch_real_cert): operand table and
  // sign masks, real_cert_tables(); null leaves that kernel unused
  const uint16_t* cwb;
  const uint32_t* cws;
  // its fold summary per channel (real_fold_switches), padded like alpha
  const float *ct1, *ct2, *cb0, *cdc;
  // where it adds the number of outputs it recomputed in the reference's
  // order (may be null)
  unsigned long long* ucnt;
  const float* alpha;   // per-channel arrays padded to a multiple of 32
  const float* A;
  const float* B;
  const float* slope;
  const float* rsign;
  int N, H, W, cin, cout;
  uint32_t* out;        // bits [N][H][W][ceil(cout/32)]; may be null
  float* f32;           // conv output [N][cout][H][W]; may be null
  // scene mode (pcols > 0): x is one cube [cin][sH][sW] cut into H x W
  // patches, pcols per row, patch n at row prow0 + n / pcols, column
  // n % pcols; a patch's rows and columns past the cube read 0
  int sH, sW, pcols, prow0;
  // v3 enc1 unit 1 (launch_react_in): the conv chain runs over ci outermost,
  // taps inside; a 1x1 projection chain runs beside it; the epilogue is
  // h = RPReLU(A*(alpha*acc) + B + proj) with A, B (= B + move1), slope
  // (= PReLU weight) and rsign (= the next tap's bias) above
  const float* pw;      // projection weights [ceil(cout/16)][chunk][4][64], see react_proj_lanes
  float* hout;          // h planes [cout][N*H*W]; of ntot patches when ntot > 0 (a batch part)
  int ntot;
  float* f32b;          // projection output [N][cout][H][W]; may be null
  // certified kernel: row parts per patch (launch_real_cert sets it)
  int rsplit;
};

// Real-conv work split: output channels per lane group and output rows per
// lane (set here so the host weight layout and the kernel agree).
#ifndef BNN_RCO
#define BNN_RCO 4
#endif
#ifndef BNN_PXR
#define BNN_PXR 2
#endif
constexpr int kRealGroup = BNN_RCO;

// host-side: int8 sign weights [cout][cin][3][3] -> [ceil(cout/G)][cin][9][G]
// floats, G = kRealGroup, zero-padded; sized real_conv_weights_len()
inline size_t real_conv_weights_len(int cout, int cin) {
  return (size_t)(cout + kRealGroup - 1) / kRealGroup * kRealGroup * cin * 9;
}
inline void real_conv_weights(const int8_t* wsign, int cout, int cin, float* out) {
  constexpr int G = kRealGroup;
  for (size_t i = 0; i < real_conv_weights_len(cout, cin); ++i) out[i] = 0.0f;
  for (int co = 0; co < cout; ++co)
    for (int ci = 0; ci < cin; ++ci)
      for (int t = 0; t < 9; ++t)
        out[(((size_t)(co / G) * cin + ci) * 9 + t) * G + co % G] = (float)wsign[((size_t)co * cin + ci) * 9 + t];
}

// Matrix-core real-conv weights, for +-1 signs only.  Input channels come
// in chunks of kRealMfmaCI (the array is zero-padded to whole chunks); per
// (16-channel group g, ci) there are three 64-bit lane masks, mask q
// holding taps 4q..4q+3: bit 16k + i is set iff w[16g + i][ci][4q + k] > 0
// (taps past 8 and channels past cout leave their bits 0).
#ifndef BNN_MCI
#define BNN_MCI 8
#endif
constexpr int kRealMfmaCI = BNN_MCI;
inline int real_conv_cin_pad(int cin) { return (cin + kRealMfmaCI - 1) / kRealMfmaCI * kRealMfmaCI; }
inline size_t real_conv_masks_len(int cout, int cin) {
  return (size_t)((cout + 15) / 16) * real_conv_cin_pad(cin) * 3;
}
inline bool real_conv_signs_only(const int8_t* wsign, int cout, int cin) {
  for (size_t i = 0; i < (size_t)cout * cin * 9; ++i)
    if (wsign[i] != 1 && wsign[i] != -1) return false;
  return true;
}
inline void real_conv_masks(const int8_t* wsign, int cout, int cin, uint64_t* out) {
  const int cp = real_conv_cin_pad(cin);
  for (size_t i = 0; i < real_conv_masks_len(cout, cin); ++i) out[i] = 0;
  for (int co = 0; co < cout; ++co)
    for (int ci = 0; ci < cin; ++ci)
      for (int t = 0; t < 9; ++t)
        if (wsign[((size_t)co * cin + ci) * 9 + t] > 0)
          out[((size_t)(co / 16) * cp + ci) * 3 + t / 4] |= 1ull << (16 * (t % 4) + co % 16);
}

// Tables of the certified first conv (all signs +-1, cin <= 128):
//  * operand table [16-channel group][wave w][tap][lane][8] fp16 bit
//    patterns: lane l holds output channel 16 g + l % 16 and, in element j,
//    input channel cin / 4 * w + 4 j + l / 16 when 4 j + l / 16 < cin / 4
//    (+1 -> 0x3C00, -1 -> 0xBC00; other elements and channels past cout -> 0);
//  * sign masks [cout padded to 16][tap][4] words: bit ci % 32 of word
//    ci / 32 set iff the weight is +1.
inline size_t real_cert_b_len(int cout) { return (size_t)((cout + 15) / 16) * 4 * 9 * 64 * 8; }
inline size_t real_cert_s_len(int cout) { return (size_t)((cout + 15) / 16) * 16 * 9 * 4; }
inline void real_cert_tables(const int8_t* wsign, int cout, int cin, uint16_t* b, uint32_t* s) {
  const int ng = (cout + 15) / 16;
  for (int g = 0; g < ng; ++g)
    for (int w = 0; w < 4; ++w)
      for (int t = 0; t < 9; ++t)
        for (int l = 0; l < 64; ++l)
          for (int j = 0; j < 8; ++j) {
            const int co = 16 * g + l % 16, cl = 4 * j + l / 16, ci = cin / 4 * w + cl;
            uint16_t v = 0;
            if (co < cout && cl < cin / 4) v = wsign[((size_t)co * cin + ci) * 9 + t] > 0 ? 0x3C00 : 0xBC00;
            b[((((size_t)g * 4 + w) * 9 + t) * 64 + l) * 8 + j] = v;
          }
  for (size_t i = 0; i < real_cert_s_len(cout); ++i) s[i] = 0;
  for (int co = 0; co < cout; ++co)
    for (int t = 0; t < 9; ++t)
      for (int ci = 0; ci < cin && ci < 128; ++ci)
        if (wsign[((size_t)co * cin + ci) * 9 + t] > 0) s[((size_t)co * 9 + t) * 4 + ci / 32] |= 1u << (ci % 32);
}
// The real fold's bit as a function of the tap sum v, in the reference's
// float steps (csrc/bnn_fold.c:62-77, A * o + B fused): o = al * v,
// z = fma(A, o, B), h = z < 0 ? sl * z : z, bit = h + rs > 0.
inline bool real_fold_bit_host(float v, float al, float A, float B, float sl, float rs) {
  const float o = al * v;
  const float z = std::fma(A, o, B);
  const float h = z < 0.0f ? sl * z : z;
  return h + rs > 0.0f;
}
// Finite floats in order as integers (-0 and +0 both 0) and back.
inline int32_t real_ford(float f) {
  uint32_t b;
  std::memcpy(&b, &f, 4);
  return (b & 0x80000000u) ? -(int32_t)(b & 0x7FFFFFFFu) : (int32_t)b;
}
inline float real_fval(int32_t o) {
  const uint32_t b = o >= 0 ? (uint32_t)o : (0x80000000u | (uint32_t)(-o));
  float f;
  std::memcpy(&f, &b, 4);
  return f;
}
// The points where the fold's bit changes along the floats of [-dc, dc]:
// there the bit of v is b0 ^ (v >= t1) ^ (v >= t2) (t = +inf: no change).
// dc is a power of two small enough that o, z, h and h + rs stay finite for
// |v| <= dc, so no step meets an infinity or a NaN.  Then z is monotone in
// v (RN products and fma are monotone), the PReLU branch splits the range
// into at most two runs, on the z >= 0 run the bit is non-decreasing in z,
// on the z < 0 run non-increasing for a negative slope and non-decreasing
// otherwise: each run holds at most one change and a slope >= 0 at most one
// in all.  Each change is found by bisection on the ordered floats, and the
// result is checked at the run ends and around every change.  Parameters
// that are not finite, or a failed check, give b0 = -1: every output of the
// channel is left to the reference-order recompute.
inline void real_fold_switches(float al, float A, float B, float sl, float rs, float* t1, float* t2, float* b0,
                               float* dc) {
  *t1 = *t2 = INFINITY;
  *b0 = -1.0f;
  *dc = 0.0f;
  const float big = 4.2535295e37f;  // 2^125 = FLT_MAX / 8, rounded down
  for (float x : {al, A, B, sl, rs})
    if (!std::isfinite(x)) return;
  const double m = std::max({1.0, std::fabs((double)al), std::fabs((double)A * al), std::fabs((double)sl * A * al)});
  if (std::fabs(B) > big || std::fabs((double)sl * B) > big || std::fabs(rs) > big) return;
  const float d = std::ldexp(1.0f, (int)std::floor(std::log2(big / m)));
  const int32_t kLo = real_ford(-d), kHi = real_ford(d);
  auto F = [&](int32_t o) { return real_fold_bit_host(real_fval(o), al, A, B, sl, rs); };
  auto Zn = [&](int32_t o) { return std::fma(A, al * real_fval(o), B) < 0.0f; };
  // first o in (a, b] where pred(o) == pred(b), given pred(a) != pred(b)
  auto bisect = [](int32_t a, int32_t b, auto pred) {
    const bool pb = pred(b);
    while ((int64_t)b - a > 1) {
      const int32_t mid = (int32_t)(((int64_t)a + b) >> 1);
      if (pred(mid) == pb) b = mid;
      else a = mid;
    }
    return b;
  };
  int32_t r1 = kHi, r2 = kHi;  // run 0 = [kLo, r1], run 1 = [r2, kHi]
  bool two = false;
  if (Zn(kLo) != Zn(kHi)) {
    r2 = bisect(kLo, kHi, Zn);
    r1 = r2 - 1;
    two = true;
  }
  std::vector<int32_t> sw;
  if (F(kLo) != F(r1)) sw.push_back(bisect(kLo, r1, F));
  if (two) {
    if (F(r1) != F(r2)) sw.push_back(r2);
    if (F(r2) != F(kHi)) sw.push_back(bisect(r2, kHi, F));
  }
  if (sw.size() > 2) return;
  const bool base = F(kLo);
  auto model = [&](int32_t o) {
    bool bit = base;
    for (int32_t t : sw) bit ^= o >= t;
    return bit;
  };
  std::vector<int32_t> probe = {kLo, kHi, r1, r2, 0, -1, 1};
  for (int32_t t : sw)
    for (int32_t k = -2; k <= 2; ++k) probe.push_back(std::min(kHi, std::max(kLo, t + k)));
  for (int32_t o : probe)
    if (model(o) != F(o)) return;
  *t1 = sw.size() > 0 ? real_fval(sw[0]) : INFINITY;
  *t2 = sw.size() > 1 ? real_fval(sw[1]) : INFINITY;
  *b0 = base ? 1.0f : 0.0f;
  *dc = d;
}
// whether launch_real_cert takes a layer of this shape (rows wider than 32
// run as tiles of 32 columns with a one-column halo either side)
inline bool real_cert_fits(int cin, int W, int rowlen) {
  return cin >= 4 && cin <= 128 && cin % 4 == 0 && W >= 4 && W % 4 == 0 && rowlen % 4 == 0;
}

// 1x1 stem weights (v2 models; signs +1, -1 or 0): 64-bit lane masks
// [group of four input channels q][16-channel group g][2]; bit 16k + i of
// mask 0 is set iff w[16g + i][4q + k] > 0, of mask 1 iff it is nonzero.
// Channels past cout or cin, and the groups that pad the group count to a
// multiple of the groups per wave, leave their bits 0.
inline int stem_groups_padded(int cout) {
  const int ngrp = (cout + 15) / 16, G = ngrp < 4 ? ngrp : 4;
  return (ngrp + G - 1) / G * G;
}
inline size_t real_stem_masks_len(int cout, int cin) { return (size_t)2 * stem_groups_padded(cout) * ((cin + 3) / 4); }
inline void real_stem_masks(const int8_t* wsign, int cout, int cin, uint64_t* out) {
  const int ngp = stem_groups_padded(cout);
  for (size_t i = 0; i < real_stem_masks_len(cout, cin); ++i) out[i] = 0;
  for (int co = 0; co < cout; ++co)
    for (int ci = 0; ci < cin; ++ci) {
      const int8_t w = wsign[(size_t)co * cin + ci];
      const size_t at = ((size_t)(ci / 4) * ngp + co / 16) * 2;
      const uint64_t bit = 1ull << (16 * (ci % 4) + co % 16);
      if (w > 0) out[at] |= bit;
      if (w != 0) out[at + 1] |= bit;
    }
}
// the 1x1 real conv + real fold (v2 stem): wm = real_stem_masks, w unused
hipError_t launch_stem(const RealArgs& a, hipStream_t s);

// v3 enc1 projection weights for the matrix-core kernel: per 16-channel
// group g and input chunk ch (kRealMfmaCI = 8 channels) four 64-float rows;
// row r < 2, lane l holds W[16g + l%16][8ch + 4r + l/16] (0 past cout/cin),
// rows 2 and 3 are 0 (one row per wave of the work group).
inline size_t react_proj_lanes_len(int cout, int cin) {
  return (size_t)((cout + 15) / 16) * (real_conv_cin_pad(cin) / kRealMfmaCI) * 4 * 64;
}
inline void react_proj_lanes(const float* W, int cout, int cin, float* out) {
  const int nch = real_conv_cin_pad(cin) / kRealMfmaCI;
  for (size_t i = 0; i < react_proj_lanes_len(cout, cin); ++i) out[i] = 0.0f;
  for (int co = 0; co < cout; ++co)
    for (int ci = 0; ci < cin; ++ci) {
      const int g = co / 16, ch = ci / kRealMfmaCI, r = (ci % kRealMfmaCI) / 4, l = 16 * (ci % 4) + co % 16;
      out[(((size_t)g * nch + ch) * 4 + r) * 64 + l] = W[(size_t)co * cin + ci];
    }
}
// v3 enc1 unit 1: 3x3 conv (lane masks) + projection + epilogue -> h planes and tap bits
hipError_t launch_react_in(const RealArgs& a, hipStream_t s);

// v3 enc1 unit 1 when its Cout is not a multiple of 8.  The reference then
// runs the general real conv (csrc/bnn_model_react.c:152-158: per output the
// taps in row-major order, each a chain over ci, then alpha * acc), which
// is the v1 order: launch_real writes that conv into `conv` first.  This
// kernel adds the projection (one fma chain over ci from +0 per output,
// csrc/bnn_react_ops.c:117-133), the real epilogue
// (csrc/bnn_react_epi.c:57-77) and the tap of unit 2, a thread per pixel.
struct ReactTailArgs {
  const float* x;      // the input, as RealArgs::x (batch, or a scene cube with the fields below)
  const float* pw;     // projection weights [cout rounded up to 16][cin], zero past cout
  const float* conv;   // alpha * conv, [N][cout][H][W]
  const float* A;      // epilogue A, B (= B + move1), slope (PReLU weight), the next tap's rsign;
  const float* B;      // padded to 32 channels
  const float* slope;
  const float* rsign;
  int N, H, W, cin, cout;
  uint32_t* out;       // tap bits [N*H*W][ceil(cout/32)]
  float* hout;         // h planes [cout][ntot*H*W], this call's first patch at column 0
  int ntot;            // patches in a plane row (0: N)
  float* f32b;         // projection output [N][cout][H][W] (debug forward); may be null
  int sH, sW, pcols, prow0;
};
hipError_t launch_react_in_tail(const ReactTailArgs& a, hipStream_t s);

// v3 1x1 projection of binary blocks (no bias), on the matrix cores:
// out[co][q] = chain over ci from 0 of W[co][ci] * x[ci][q] over the planes
// of x (q = (n*H + y)*W + x).  With x1 set, channels >= c0 come from the
// nearest-2x upsample of x1 (planes at h1 x w1) placed at (oh, ow); positions
// it does not cover read 0.  Weights as react_pw_lanes lays them out.
struct ProjArgs {
  const float* x0;      // planes [c0][N*H*W]
  const float* x1;      // planes [cin-c0][N*h1*w1], or null
  int c0, cin, cout;
  int N, H, W, h1, w1, oh, ow, uh, uw;
  const float* w;       // react_pw_lanes layout
  float* out;           // planes [cout][N*H*W]
  // a batch part: every plane holds ntot patches, this call N of them from
  // patch n0, x0/x1/out already moved to n0 (ntot 0: the whole batch)
  int ntot, n0;
};
// [ceil(cout/16)][ceil(cin/4)][64]: lane l of quad q holds W[16g + l%16][4q + l/16]
inline size_t react_pw_lanes_len(int cout, int cin) { return (size_t)((cout + 15) / 16) * ((cin + 3) / 4) * 64; }
inline void react_pw_lanes(const float* W, int cout, int cin, float* out) {
  const int nq = (cin + 3) / 4;
  for (size_t i = 0; i < react_pw_lanes_len(cout, cin); ++i) out[i] = 0.0f;
  for (int co = 0; co < cout; ++co)
    for (int ci = 0; ci < cin; ++ci)
      out[(((size_t)(co / 16) * nq + ci / 4) * 64) + 16 * (ci % 4) + co % 16] = W[(size_t)co * cin + ci];
}
hipError_t launch_proj(const ProjArgs& a, hipStream_t s);

// v3 batch-1 kernel ABI helpers (one thread per output element)
hipError_t launch_react_epi(const void* acc, int kind, const float* res, float* out, int C, long HW,
                            const float* A, const float* B, const float* move1, const float* prelu_w, int form,
                            hipStream_t s);
hipError_t launch_react_tap(const float* x, int8_t* out, int C, long HW, const float* rsign, hipStream_t s);
hipError_t launch_maxpool_real(const float* x, float* out, int C, int H, int W, int k, int stride, hipStream_t s);
hipError_t launch_conv3_chain(const float* x, const int8_t* wsign, const float* alpha, float* out, int cin, int H,
                              int W, int cout, hipStream_t s);

// Launchers return hipSuccess or the first launch error.  mt = micro-tile
// side (1 or 2), cog = output channels per work-item (8/16/32).
hipError_t launch_bconv(const BconvArgs& a, int epi, int mt, int cog, bool dump,
                        hipStream_t s);

// Binary conv on the int8 matrix cores (v_mfma_i32_16x16x64_i8), for
// cout % 64 == 0 and the EPI_FOLD / EPI_POOL epilogues.  With activation
// bits alpha in {0,1} (0 for taps outside the image) and weights w in
// {-1,+1}, D = sum over valid taps of w*alpha and
//   P = sum over valid taps of w*(2*alpha - 1) = 2*D - S,
// S = sum of w over the valid taps, which depends only on which taps are
// valid: 16 border classes (row pattern x column pattern, each of: all
// valid, first invalid, last invalid, both invalid).  K runs over chunks of
// two activation words (64 channels) of one input segment, a concat's
// upsampled segment after the first (an odd segment's last chunk has an
// empty second word); within a chunk over the 9 taps, and within a tap over
// the two words: pair (chunk * 9 + tap) * 2 + word, 32 channels each.
struct MfmaConv {
  const int8_t* w;      // [coutp][npair][32] int8, +-1, 0 for padded channels and empty words
  const int32_t* s;     // [16][coutp] S per border class
  int npair;
};
inline int mfma_nchunk(int cw0, int cw1) { return (cw0 + 1) / 2 + (cw1 + 1) / 2; }
inline int mfma_npair(int cw0, int cw1) { return 18 * mfma_nchunk(cw0, cw1); }
// kidx sign bits -> the int8 weight table; channel layout as repack_bin
// (a concat's upsampled channels start at word cw0)
inline void mfma_conv_tables(const uint64_t* kbits, int cin, int cout, int cs, int8_t* w, int32_t* stab) {
  const int cw0 = (cs ? cs : cin) / 32 + ((cs ? cs : cin) % 32 != 0);
  const int cw1 = cs ? (cin - cs + 31) / 32 : 0;
  const int npair = mfma_npair(cw0, cw1), nc0 = (cw0 + 1) / 2;
  const int coutp = (cout + 63) / 64 * 64, nw = (cin * 9 + 63) / 64;
  for (size_t i = 0; i < (size_t)coutp * npair * 32; ++i) w[i] = 0;
  std::vector<long> T((size_t)coutp * 9, 0);
  for (int co = 0; co < cout; ++co)
    for (int ci = 0; ci < cin; ++ci) {
      int wd, b, c;  // word within its segment, bit, chunk
      if (!cs || ci < cs) { wd = ci >> 5; b = ci & 31; c = wd >> 1; }
      else { wd = (ci - cs) >> 5; b = (ci - cs) & 31; c = nc0 + (wd >> 1); }
      for (int t = 0; t < 9; ++t) {
        const int k = ci * 9 + t;
        const int v = ((kbits[(size_t)co * nw + (k >> 6)] >> (k & 63)) & 1ull) ? 1 : -1;
        const int pr = (c * 9 + t) * 2 + (wd & 1);
        w[((size_t)co * npair + pr) * 32 + b] = (int8_t)v;
        T[(size_t)co * 9 + t] += v;
      }
    }
  // valid rows / columns of the 3x3 window for patterns 0..3
  static const int valid[4][3] = {{1, 1, 1}, {0, 1, 1}, {1, 1, 0}, {0, 1, 0}};
  for (int rp = 0; rp < 4; ++rp)
    for (int cp = 0; cp < 4; ++cp)
      for (int co = 0; co < coutp; ++co) {
        long sum = 0;
        for (int ky = 0; ky < 3; ++ky)
          for (int kx = 0; kx < 3; ++kx)
            if (valid[rp][ky] && valid[cp][kx]) sum += T[(size_t)co * 9 + ky * 3 + kx];
        stab[(size_t)(rp * 4 + cp) * coutp + co] = (int32_t)sum;
      }
}
inline size_t mfma_w_len(int cin, int cout, int cs) {
  const int cw0 = ((cs ? cs : cin) + 31) / 32, cw1 = cs ? (cin - cs + 31) / 32 : 0;
  return (size_t)(cout + 63) / 64 * 64 * mfma_npair(cw0, cw1) * 32;
}
inline size_t mfma_s_len(int cout) { return (size_t)16 * ((cout + 63) / 64 * 64); }
// Whether launch_bconv_mfma takes a layer of this shape (cout % 64 == 0 and
// an image narrow enough for its LDS tile).
bool mfma_conv_fits(int cout, int H, int W, int epi);
hipError_t launch_bconv_mfma(const BconvArgs& a, const MfmaConv& m, int epi, bool dump, hipStream_t s);
hipError_t launch_real(const RealArgs& a, hipStream_t s);

// Simple kernels behind the reference's batch-1 kernel ABI.
hipError_t launch_pack_act(const int8_t* a, uint32_t* out, int N, int C, int H, int W,
                           hipStream_t s);
hipError_t launch_bconv_generic(const uint32_t* act, const uint32_t* wt, int32_t* P,
                                int cin, int H, int W, int cout, int kh, int kw,
                                int pad, int stride, hipStream_t s);
hipError_t launch_bconv_naive(const int8_t* a, const int8_t* w, int32_t* P, int cin,
                              int H, int W, int cout, int kh, int kw, int pad,
                              int stride, hipStream_t s);
hipError_t launch_real_generic(const float* x, const float* w, const float* alpha,
                               float* out, int cin, int H, int W, int cout, int kh,
                               int kw, int pad, int stride, hipStream_t s);
hipError_t launch_maxpool(const int32_t* P, int32_t* out, int C, int H, int W, int k,
                          int stride, hipStream_t s);
hipError_t launch_fold_int(const int32_t* P, int8_t* out, int C, int HW,
                           const int32_t* type, const int32_t* t, const int32_t* lo,
                           const int32_t* hi, hipStream_t s);
hipError_t launch_fold_real(const float* x, int8_t* out, int C, int HW, const float* A,
                            const float* B, const float* slope, const float* rsign,
                            hipStream_t s);
// The middle of the v1 UNet for patches whose level 2 is 8 x 8 (32-35 px):
// enc3.c1, enc3.c2 (+pool), enc4.c1, enc4.c2 (+pool), bott.c1, bott.c2,
// dec4.c1 (concat), dec4.c2, dec3.c1 (concat), dec3.c2 in one kernel, one
// block per patch (bnn_mid.hip).  Per layer: weights [words][9 taps][coutp]
// (coutp = cout rounded up to 64, zero past cout; a concat's words are the
// skip's, then the upsampled tensor's), the fold as canonical intervals
// (lo, wid) padded to coutp with wid 0, the pool layers' second rule, and
// the P dumps of the debug forward.
constexpr int kMidLayers = 10, kMidTensors = 13;
struct MidLayer {
  const uint32_t* w;
  const int32_t* lo;
  const uint32_t* wid;
  const int32_t* lo2;
  const uint32_t* wid2;
  int cin, cout;
  int32_t* P;   // [N][cout][d][d] (debug forward)
  int32_t* P2;  // pooled P (debug forward, pool layers)
};
// The level-1 layers around the middle (ext = 1, patches whose level 1 is
// 16 x 16 and whose level-1 layers have at most 32 output channels):
// enc2.c1, enc2.c2 (+pool, into tensor 0), dec2.c1 (concat of the enc2 skip
// and tensor 12), dec2.c2, pixels on lanes.  Weights in k_bconv's table
// ([word][cout rounded to 32][9], the first segment's taps paired when
// pair), rules padded to 64 with width 0.
constexpr int kMidXLayers = 4, kMidXTensors = 5;
struct MidXLayer {
  const uint32_t* w;
  const int32_t* lo;
  const uint32_t* wid;
  const int32_t* lo2;
  const uint32_t* wid2;
  int cin, cout, cw0, cw1, pair;
  int32_t* P;   // [N][cout][16][16] (debug forward)
  int32_t* P2;  // pooled P (debug forward, enc2.c2)
};
// Tensors, [N][d][d][cw] words each: 0 enc2 pooled bits (input), 1 enc3.c1,
// 2 enc3 skip, 3 enc3 down, 4 enc4.c1, 5 enc4 skip, 6 enc4 down, 7 bott.c1,
// 8 bott.c2, 9 dec4.c1, 10 dec4.c2, 11 dec3.c1, 12 dec3.c2 (output).  off: a
// tensor's word offset in the block's LDS (one patch), ldsw the total.
// With ext, tensor 0 is made in the kernel and the level-1 tensors are
// 0 enc1 pooled bits (input), 1 enc2.c1, 2 enc2 skip, 3 dec2.c1, 4 dec2.c2
// (output), 16 x 16 each.
struct MidArgs {
  MidLayer L[kMidLayers];
  uint32_t* t[kMidTensors];
  int off[kMidTensors], dim[kMidTensors], cw[kMidTensors];
  int N, ldsw;
  int ext;
  MidXLayer X[kMidXLayers];
  uint32_t* xt[kMidXTensors];
  int xoff[kMidXTensors], xcw[kMidXTensors];
};
hipError_t launch_mid(const MidArgs& a, bool dump, hipStream_t s);

// the certified first conv (bits only; RealArgs with cwb, cws, out, no f32)
hipError_t launch_real_cert(const RealArgs& a, hipStream_t s);
// how many patches of this shape one round of the certified kernel holds
// (its blocks resident on the device at once), 0 if it cannot tell
long real_cert_round(int cin, int cout, int W);

// The 1x1 head as its own kernel (heads over more than 32 channels, which
// one epilogue group cannot hold): input the head layer's packed bits
// [N][H][W][cw] read as +-1 (v1), or its float planes (v3: element
// (c, n, y, x) at c * plane + (n * H + y) * W + x, bits null).
struct HeadArgs {
  const uint32_t* bits;
  int cw;
  const float* planes;
  size_t plane;
  int cin;
  const float* hw;  // [ncls][cin]
  const float* hb;  // [ncls]
  int ncls;
  float* logits;    // [N][ncls][H][W], or the scene map [ncls][sH][sW]
  int N, H, W;
  int sH, sW, pcols, prow0;  // scene mode (pcols > 0), as in RealArgs
};
hipError_t launch_head_sep(const HeadArgs& a, hipStream_t s);

hipError_t launch_head(const float* a, const float* W, const float* b, float* out,
                       int cin, int HW, int cout, hipStream_t s);

}  // namespace bnn
