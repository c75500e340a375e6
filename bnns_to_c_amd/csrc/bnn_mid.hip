// bnn_mid.hip - the middle of the v1 UNet for 32 x 32 patches in one kernel:
// enc3 (8x8), enc4 (4x4), the bottleneck (2x2), dec4 (4x4) and dec3 (8x8),
// ten binary convs with their folds, both 2x2 max-pools on P and both
// nearest-upsample concats (csrc/bnn_model.c:190-235), one block per patch.
//
// At these sizes a patch has far more channels than pixels (64 pixels and 64
// channels at 8x8, 4 pixels and 256 channels at 2x2), so lanes hold output
// channels, not pixels: lane l of a wave is output channel 64 g + l of its
// channel group g, and its weights for the current input word (nine taps)
// sit in registers.  The patch's activations live in LDS; an input word is
// read once (the same address for every lane, a broadcast) and added into
// each of the up to nine outputs it feeds, one XOR + popcount each:
//   P[p] = Cin * taps_valid(p) - 2 * sum over valid taps, words of
//          popcount(a ^ w)
// which is the reference's xnor-popcount P (csrc/bnn_conv.c:23-36): taps
// outside the image are never visited.  Tail bits past Cin are 0 in both the
// activations and the weights.  The fold is the canonical interval rule
// (bit = (uint32)(P - lo) < wid, csrc/bnn_fold.c:37-60); a pool layer also
// takes the 2x2 floor-mode max of P and its second rule
// (csrc/bnn_maxpool.c:28-48).  The bits of a pixel's 64 channels are one
// ballot.
//
// In LDS a tensor is planar by word (word w of pixel (y, x) at
// off + (w * d + y) * d + x), so one input row of one word is d consecutive
// words: two 128-bit reads at 8 x 8.  The rows of the next word are read
// while the current word's popcounts run.  The four waves split each layer
// into (channel group, band of two output rows) units; between layers the
// block synchronises; at the end the last layer's output (and, for the debug
// forward, every intermediate tensor) is written to the workspace in its
// usual [N][h][w][words] layout.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bnn_device.h"
#include "bnn_kernels.h"

namespace bnn {
namespace {

__device__ __forceinline__ uint32_t mid_bcnt(uint32_t x, uint32_t acc) {
  uint32_t r;
  asm("v_bcnt_u32_b32 %0, %1, %2" : "=v"(r) : "v"(x), "v"(acc));
  return r;
}

// LDS tensor: word w of position (y, x) at off + (w * d + y) * d + x
struct MidT {
  int off, d, cw;
};

// K consecutive LDS words from p (p 4 K bytes aligned for K = 2, 4, 8)
template <int K>
__device__ __forceinline__ void lds_row(const uint32_t* p, uint32_t (&r)[K]) {
  if constexpr (K == 8) {
    const uint4 a = reinterpret_cast<const uint4*>(p)[0], b = reinterpret_cast<const uint4*>(p)[1];
    r[0] = a.x; r[1] = a.y; r[2] = a.z; r[3] = a.w;
    r[4] = b.x; r[5] = b.y; r[6] = b.z; r[7] = b.w;
  } else if constexpr (K == 4) {
    const uint4 a = reinterpret_cast<const uint4*>(p)[0];
    r[0] = a.x; r[1] = a.y; r[2] = a.z; r[3] = a.w;
  } else {
    static_assert(K == 2, "row width");
    const uint2 a = reinterpret_cast<const uint2*>(p)[0];
    r[0] = a.x; r[1] = a.y;
  }
}

// The input rows r0 - 1 .. r0 + RB of word w (D wide; rows outside the image
// are not read).  UP: the word of a D/2 x D/2 tensor through the nearest 2x
// upsample, row qy reading source row qy / 2.
template <int D, int RB, bool UP>
__device__ __forceinline__ void load_rows(const uint32_t* lds, MidT t, int w, int r0, uint32_t (&rows)[RB + 2][D]) {
  constexpr int S = UP ? D / 2 : D;
#pragma unroll
  for (int qr = -1; qr <= RB; ++qr) {
    const int qy = r0 + qr;
    if ((qr < 0 || qr >= RB) && (qy < 0 || qy >= D)) continue;
    uint32_t r[S];
    lds_row<S>(lds + t.off + (w * S + (UP ? qy >> 1 : qy)) * S, r);
#pragma unroll
    for (int x = 0; x < D; ++x) rows[qr + 1][x] = r[UP ? x >> 1 : x];
  }
}

// The popcounts of one input word into the band's accumulators.
template <int D, int RB>
__device__ __forceinline__ void word_step(const uint32_t (&rows)[RB + 2][D], const uint32_t (&wt)[9], int r0,
                                          uint32_t (&acc)[RB][D]) {
#pragma unroll
  for (int qr = -1; qr <= RB; ++qr) {
    const int qy = r0 + qr;
    if ((qr < 0 || qr >= RB) && (qy < 0 || qy >= D)) continue;
#pragma unroll
    for (int qx = 0; qx < D; ++qx) {
      const uint32_t a = rows[qr + 1][qx];
#pragma unroll
      for (int ky = 0; ky < 3; ++ky) {
        const int pr = qr - ky + 1;  // output row, relative to r0
        if (pr < 0 || pr >= RB) continue;
#pragma unroll
        for (int kx = 0; kx < 3; ++kx) {
          const int px = qx - kx + 1;
          if (px < 0 || px >= D) continue;
          acc[pr][px] = mid_bcnt(a ^ wt[ky * 3 + kx], acc[pr][px]);
        }
      }
    }
  }
}

// Word w's input rows and its nine weights (wbase + w * wstride + 64 t: the
// table is [word][channel group][tap][64 lanes], so the taps are immediate
// offsets from one address).
template <int D, int RB, bool UP>
__device__ __forceinline__ void load_word(const uint32_t* lds, MidT src, const uint32_t* wbase, int wstride, int w,
                                          int r0, uint32_t (&rows)[RB + 2][D], uint32_t (&wt)[9]) {
  load_rows<D, RB, UP>(lds, src, w, r0, rows);
  const uint32_t* wp = wbase + (size_t)w * wstride;
#pragma unroll
  for (int t = 0; t < 9; ++t) wt[t] = wp[t * 64];
}

// The words of one source tensor (src.cw of them), the rows and weights of
// the next word loaded while the current one is counted.  Two register sets,
// so that the prefetch needs no copies: word w counts from set A while w + 1
// loads into B, then the other way round.
template <int D, int RB, bool UP>
__device__ __forceinline__ void src_words(const uint32_t* lds, MidT src, const uint32_t* wbase, int wstride, int r0,
                                          uint32_t (&acc)[RB][D]) {
  uint32_t ra[RB + 2][D], rb[RB + 2][D], wa[9], wb[9];
  load_word<D, RB, UP>(lds, src, wbase, wstride, 0, r0, ra, wa);
  int w = 0;
#pragma unroll 1
  for (; w + 1 < src.cw; w += 2) {
    load_word<D, RB, UP>(lds, src, wbase, wstride, w + 1, r0, rb, wb);
    word_step<D, RB>(ra, wa, r0, acc);
    if (w + 2 < src.cw) load_word<D, RB, UP>(lds, src, wbase, wstride, w + 2, r0, ra, wa);
    word_step<D, RB>(rb, wb, r0, acc);
  }
  if (w < src.cw) word_step<D, RB>(ra, wa, r0, acc);
}

// One conv of the middle: output dims D x D (stride 1, pad 1), input src0
// (D x D) and, for a concat, src1 (D/2 x D/2) read through the nearest 2x
// upsample.  The calling wave computes channel group cg (lanes = channels
// 64 cg ..) for output rows [r0, r0 + RB).  Results: bits into dst (and,
// POOL, the pooled rule's bits into dst2 at D/2 x D/2).
template <int D, int RB, bool POOL, bool CAT, bool DUMP>
__device__ __forceinline__ void mid_unit(const MidLayer& L, uint32_t* lds, MidT src0, MidT src1, MidT dst,
                                         MidT dst2, int cg, int r0, int n, int lane) {
  const int co = cg * 64 + lane;
  const int wstride = (L.cout + 63) / 64 * 9 * 64;  // words per input word of the table
  uint32_t acc[RB][D];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < D; ++j) acc[i][j] = 0u;
  // this lane's weights: [word][channel group][tap][64]
  const uint32_t* wbase = L.w + cg * 9 * 64 + lane;
  // the rule(s), padded to coutp with width 0 (bit 0 past cout)
  const int32_t lo = L.lo[co];
  const uint32_t wid = L.wid[co];
  int32_t lo2 = 0;
  uint32_t wid2 = 0u;
  if constexpr (POOL) { lo2 = L.lo2[co]; wid2 = L.wid2[co]; }
  src_words<D, RB, false>(lds, src0, wbase, wstride, r0, acc);
  if constexpr (CAT) src_words<D, RB, true>(lds, src1, wbase + (size_t)src0.cw * wstride, wstride, r0, acc);
  // epilogue: P, the rule, one ballot per pixel
  const bool live = co < L.cout;
  const int wi = cg * 2 + (lane & 1);
  int32_t P[RB][D];
#pragma unroll
  for (int i = 0; i < RB; ++i) {
    const int py = r0 + i;
    const int rows = 1 + (py > 0 ? 1 : 0) + (py < D - 1 ? 1 : 0);
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const int cols = 1 + (j > 0 ? 1 : 0) + (j < D - 1 ? 1 : 0);
      P[i][j] = L.cin * rows * cols - 2 * (int32_t)acc[i][j];
      if (DUMP && live) L.P[((size_t)n * L.cout + co) * (D * D) + py * D + j] = P[i][j];
      const bool bit = (uint32_t)P[i][j] - (uint32_t)lo < wid;
      const uint64_t m = __builtin_amdgcn_ballot_w64(bit);
      if (lane < 2 && wi < dst.cw) lds[dst.off + (wi * D + py) * D + j] = lane ? (uint32_t)(m >> 32) : (uint32_t)m;
    }
  }
  if constexpr (POOL) {
    constexpr int H = D / 2;
#pragma unroll
    for (int i = 0; i + 1 < RB; i += 2) {
      const int yy = (r0 + i) >> 1;
#pragma unroll
      for (int j = 0; j + 1 < D; j += 2) {
        const int32_t pm = max(max(P[i][j], P[i][j + 1]), max(P[i + 1][j], P[i + 1][j + 1]));
        if (DUMP && live) L.P2[((size_t)n * L.cout + co) * (H * H) + yy * H + (j >> 1)] = pm;
        const bool bit = (uint32_t)pm - (uint32_t)lo2 < wid2;
        const uint64_t m = __builtin_amdgcn_ballot_w64(bit);
        if (lane < 2 && wi < dst2.cw)
          lds[dst2.off + (wi * H + yy) * H + (j >> 1)] = lane ? (uint32_t)(m >> 32) : (uint32_t)m;
      }
    }
  }
}

// Bands of two output rows: a layer is (channel group, band) units over the
// four waves, a channel group taking D / 2 bands.  For the base-16 UNet
// that keeps all four waves busy in every layer (64 channels at 8x8: 4
// bands; 128 at 4x4: 2 groups x 2 bands; 256 at 2x2: 4 groups x 1 band).
// The host takes this kernel only for widths that keep the work within one
// or two passes (mid_fits), and the per-layer kernels otherwise.
template <int D, bool POOL, bool CAT, bool DUMP>
__device__ __forceinline__ void mid_layer(const MidLayer& L, uint32_t* lds, MidT src0, MidT src1, MidT dst,
                                          MidT dst2, int n, int wv, int lane) {
  const int ncg = (L.cout + 63) / 64;
  constexpr int nband = D / 2;
  for (int u = wv; u < ncg * nband; u += 4) {
    const int cg = u / nband, r0 = (u - cg * nband) * 2;
    mid_unit<D, 2, POOL, CAT, DUMP>(L, lds, src0, src1, dst, dst2, cg, r0, n, lane);
  }
  __syncthreads();
}

// ---- level 1 (16 x 16), pixels on lanes -------------------------------
// At 16 x 16 a patch has 256 pixels and at most 32 channels per layer here,
// so thread t of the block holds one pixel and all 32 output channels: the
// pixel of quad q = t / 4 (quads of 2 x 2 pixels, row by row) at
// y = 2 (q / 8) + (t / 2) % 2, x = 2 (q % 8) + t % 2, so that a pool's four
// pixels are four consecutive lanes.  A channel's weights are the same for
// every lane (scalar loads from k_bconv's [word][channel][tap] table), an
// input word's 3 x 3 window is nine LDS reads, and a tap outside the image
// reads the pixel's own word under a zero mask: (a ^ w) & m, one v_bitop3.
// P = Cin * taps_valid - 2 * sum popcount, as in the rest of the kernel.
typedef const __attribute__((address_space(4))) uint32_t* mid_cu32;
typedef const __attribute__((address_space(4))) int32_t* mid_ci32;

template <int D>
struct PxWin {
  uint32_t o[9], u[9], m[9];  // window offsets (D x D plane, upsampled D/2 plane), masks
  int nvalid;
};

template <int D, bool CAT>
__device__ __forceinline__ void px_window(int y, int x, PxWin<D>& g) {
  bool rv[3], cv[3];
  int ry[3], cx[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const int iy = y + k - 1, ix = x + k - 1;
    rv[k] = (uint32_t)iy < (uint32_t)D;
    cv[k] = (uint32_t)ix < (uint32_t)D;
    ry[k] = rv[k] ? iy : y;
    cx[k] = cv[k] ? ix : x;
  }
#pragma unroll
  for (int ky = 0; ky < 3; ++ky)
#pragma unroll
    for (int kx = 0; kx < 3; ++kx) {
      const int t = ky * 3 + kx;
      g.o[t] = (uint32_t)(ry[ky] * D + cx[kx]);
      g.m[t] = rv[ky] && cv[kx] ? ~0u : 0u;
      if constexpr (CAT) g.u[t] = (uint32_t)((ry[ky] >> 1) * (D / 2) + (cx[kx] >> 1));
    }
  g.nvalid = ((int)rv[0] + (int)rv[1] + (int)rv[2]) * ((int)cv[0] + (int)cv[1] + (int)cv[2]);
}

// one input word's window into the 32 counts; the weights of 4 channels
// (36 words) come as one batch of scalar loads
__device__ __forceinline__ void px_word(uint32_t (&acc)[32], const uint32_t (&a)[9], const uint32_t (&m)[9],
                                        mid_cu32 wr) {
#pragma unroll
  for (int j0 = 0; j0 < 32; j0 += 4) {
    uint32_t w9[4][9];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
#pragma unroll
      for (int t = 0; t < 9; ++t) w9[jj][t] = wr[(j0 + jj) * 9 + t];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      uint32_t d = acc[j0 + jj];
#pragma unroll
      for (int t = 0; t < 9; ++t) d = mid_bcnt((a[t] ^ w9[jj][t]) & m[t], d);
      acc[j0 + jj] = d;
    }
  }
}

// the same for an input of at most 16 channels: taps 2p and 2p + 1 packed
// in one word (low and high half), tap 8 alone, weights [channel][5]
__device__ __forceinline__ void px_pair(uint32_t (&acc)[32], const uint32_t (&a)[9], const uint32_t (&m)[9],
                                        mid_cu32 wr) {
  uint32_t c[5], mm[5];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    c[q] = a[2 * q] | (a[2 * q + 1] << 16);
    mm[q] = (m[2 * q] & 0xFFFFu) | (m[2 * q + 1] & 0xFFFF0000u);
  }
  c[4] = a[8];
  mm[4] = m[8];
#pragma unroll
  for (int j0 = 0; j0 < 32; j0 += 8) {
    uint32_t w5[8][5];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj)
#pragma unroll
      for (int q = 0; q < 5; ++q) w5[jj][q] = wr[(j0 + jj) * 5 + q];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      uint32_t d = acc[j0 + jj];
#pragma unroll
      for (int q = 0; q < 5; ++q) d = mid_bcnt((c[q] ^ w5[jj][q]) & mm[q], d);
      acc[j0 + jj] = d;
    }
  }
}

// the max of v over the lane's quad (lanes 4k .. 4k + 3)
__device__ __forceinline__ int32_t quad_max(int32_t v) {
  v = max(v, __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false));  // quad_perm [1, 0, 3, 2]
  return max(v, __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false));  // quad_perm [2, 3, 0, 1]
}

// One level-1 conv (stride 1, pad 1, D x D): input src0 and, CAT, src1
// (D/2 x D/2) through the nearest 2x upsample; output bits into dst and,
// POOL, the pooled rule's bits into dst2.  Every thread of the block takes
// part; the block synchronises at the end.
template <int D, bool POOL, bool CAT, bool DUMP>
__device__ __forceinline__ void px_layer(const MidXLayer& L, uint32_t* lds, MidT src0, MidT src1, MidT dst,
                                         MidT dst2, int n, int t) {
  constexpr int H2 = D / 2, NP = D * D;
  static_assert(NP == 256, "one pixel per thread");
  // (an opaque copy of t: the window is recomputed per layer instead of
  // being held in registers through the middle's layers)
  asm volatile("" : "+v"(t));
  const int q = t >> 2;
  const int y = 2 * (q / H2) + ((t >> 1) & 1), x = 2 * (q % H2) + (t & 1);
  PxWin<D> g;
  px_window<D, CAT>(y, x, g);
  uint32_t acc[32];
#pragma unroll
  for (int j = 0; j < 32; ++j) acc[j] = 0u;
  const mid_cu32 wt = (mid_cu32)L.w;
  const int coutp = (L.cout + 31) & ~31;
  size_t seg1;
  if (L.pair) {
    uint32_t a9[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) a9[k] = lds[src0.off + g.o[k]];
    px_pair(acc, a9, g.m, wt);
    seg1 = (size_t)coutp * 5;
  } else {
#pragma unroll 1
    for (int w = 0; w < L.cw0; ++w) {
      uint32_t a9[9];
#pragma unroll
      for (int k = 0; k < 9; ++k) a9[k] = lds[src0.off + w * NP + g.o[k]];
      px_word(acc, a9, g.m, wt + (size_t)w * coutp * 9);
    }
    seg1 = (size_t)L.cw0 * coutp * 9;
  }
  if constexpr (CAT) {
#pragma unroll 1
    for (int w = 0; w < L.cw1; ++w) {
      uint32_t a9[9];
#pragma unroll
      for (int k = 0; k < 9; ++k) a9[k] = lds[src1.off + w * (H2 * H2) + g.u[k]];
      px_word(acc, a9, g.m, wt + seg1 + (size_t)w * coutp * 9);
    }
  }
  // epilogue: P, the rule (and the pool's max and second rule), one word
  const mid_ci32 lo = (mid_ci32)L.lo;
  const mid_cu32 wid = (mid_cu32)L.wid;
  const int32_t base = L.cin * g.nvalid;
  uint32_t bits = 0u, b2 = 0u;
  const bool lead = (t & 3) == 0;
  const int pp = (y >> 1) * H2 + (x >> 1);
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    const int32_t P = base - 2 * (int32_t)acc[j];
    bits |= ((uint32_t)P - (uint32_t)lo[j] < wid[j] ? 1u : 0u) << j;
    if (DUMP && j < L.cout) L.P[((size_t)n * L.cout + j) * NP + y * D + x] = P;
    if constexpr (POOL) {
      const int32_t pm = quad_max(P);
      b2 |= ((uint32_t)pm - (uint32_t)((mid_ci32)L.lo2)[j] < ((mid_cu32)L.wid2)[j] ? 1u : 0u) << j;
      if (DUMP && lead && j < L.cout) L.P2[((size_t)n * L.cout + j) * (H2 * H2) + pp] = pm;
    }
  }
  lds[dst.off + y * D + x] = bits;
  if (POOL && lead) lds[dst2.off + pp] = b2;
  __syncthreads();
}

// [N][d][d][cw] words at src (patch n) into LDS, planar by word
__device__ __forceinline__ void mid_load(uint32_t* lds, MidT t, const uint32_t* src, int n, int tid) {
  const int np = t.d * t.d, nw = np * t.cw;
  src += (size_t)n * nw;
  for (int k = tid; k < nw; k += 256) {
    const int w = k / np, p = k - w * np;
    lds[t.off + k] = src[p * t.cw + w];
  }
}
// and back
__device__ __forceinline__ void mid_store(const uint32_t* lds, MidT t, uint32_t* dst, int n, int tid) {
  const int np = t.d * t.d, nw = np * t.cw;
  dst += (size_t)n * nw;
  for (int k = tid; k < nw; k += 256) {
    const int p = k / t.cw, w = k - p * t.cw;
    dst[k] = lds[t.off + w * np + p];
  }
}

template <bool DUMP, bool EXT>
__global__ __launch_bounds__(256) void k_mid(const MidArgs a) {
  extern __shared__ uint32_t mlds[];
  const int n = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  MidT T[kMidTensors];
#pragma unroll
  for (int i = 0; i < kMidTensors; ++i) T[i] = MidT{a.off[i], a.dim[i], a.cw[i]};
  const MidT none{0, 0, 0};
  MidT X[kMidXTensors];
#pragma unroll
  for (int i = 0; i < kMidXTensors; ++i) X[i] = MidT{a.xoff[i], 16, a.xcw[i]};
  if constexpr (EXT) {
    // enc1's pooled bits (16 x 16) in; enc2.c1 and enc2.c2, whose pool
    // makes tensor 0
    mid_load(mlds, X[0], a.xt[0], n, tid);
    __syncthreads();
    px_layer<16, false, false, DUMP>(a.X[0], mlds, X[0], none, X[1], none, n, tid);  // enc2.c1
    px_layer<16, true, false, DUMP>(a.X[1], mlds, X[1], none, X[2], T[0], n, tid);   // enc2.c2
  } else {
    // the input (enc2's pooled bits, 8 x 8)
    mid_load(mlds, T[0], a.t[0], n, tid);
    __syncthreads();
  }
  mid_layer<8, false, false, DUMP>(a.L[0], mlds, T[0], none, T[1], none, n, wv, lane);   // enc3.c1
  mid_layer<8, true, false, DUMP>(a.L[1], mlds, T[1], none, T[2], T[3], n, wv, lane);    // enc3.c2
  mid_layer<4, false, false, DUMP>(a.L[2], mlds, T[3], none, T[4], none, n, wv, lane);   // enc4.c1
  mid_layer<4, true, false, DUMP>(a.L[3], mlds, T[4], none, T[5], T[6], n, wv, lane);    // enc4.c2
  mid_layer<2, false, false, DUMP>(a.L[4], mlds, T[6], none, T[7], none, n, wv, lane);   // bott.c1
  mid_layer<2, false, false, DUMP>(a.L[5], mlds, T[7], none, T[8], none, n, wv, lane);   // bott.c2
  mid_layer<4, false, true, DUMP>(a.L[6], mlds, T[5], T[8], T[9], none, n, wv, lane);    // dec4.c1
  mid_layer<4, false, false, DUMP>(a.L[7], mlds, T[9], none, T[10], none, n, wv, lane);  // dec4.c2
  mid_layer<8, false, true, DUMP>(a.L[8], mlds, T[2], T[10], T[11], none, n, wv, lane);  // dec3.c1
  mid_layer<8, false, false, DUMP>(a.L[9], mlds, T[11], none, T[12], none, n, wv, lane); // dec3.c2
  if constexpr (EXT) {
    px_layer<16, false, true, DUMP>(a.X[2], mlds, X[2], T[12], X[3], none, n, tid);  // dec2.c1
    px_layer<16, false, false, DUMP>(a.X[3], mlds, X[3], none, X[4], none, n, tid);  // dec2.c2
    // out: dec2.c2's bits; the debug forward also takes every intermediate
    if (DUMP) {
#pragma unroll 1
      for (int i = 0; i < kMidTensors; ++i) mid_store(mlds, T[i], a.t[i], n, tid);
#pragma unroll 1
      for (int i = 1; i < kMidXTensors - 1; ++i) mid_store(mlds, X[i], a.xt[i], n, tid);
    }
    mid_store(mlds, X[kMidXTensors - 1], a.xt[kMidXTensors - 1], n, tid);
  } else {
    // out: dec3.c2's bits; the debug forward also takes every intermediate
#pragma unroll 1
    for (int i = DUMP ? 1 : kMidTensors - 1; i < kMidTensors; ++i) mid_store(mlds, T[i], a.t[i], n, tid);
  }
}

}  // namespace

hipError_t launch_mid(const MidArgs& a, bool dump, hipStream_t s) {
  if (a.N <= 0) return hipSuccess;
  const bool ext = a.ext != 0;
  for (int i = 0; i < kMidTensors; ++i) {
    // (with ext, tensor 0 is made in the kernel and tensor 12 stays there)
    const bool need = dump || (ext ? false : i == 0 || i == kMidTensors - 1);
    if (!a.t[i] && need) return hipErrorInvalidValue;
    // 128-bit row reads: every tensor starts on 4 words
    if (a.off[i] % 4) return hipErrorInvalidValue;
  }
  if (dump)
    for (int l = 0; l < kMidLayers; ++l)
      if (!a.L[l].P || ((l == 1 || l == 3) && !a.L[l].P2)) return hipErrorInvalidValue;
  if (ext) {
    for (int i = 0; i < kMidXTensors; ++i)
      if (!a.xt[i] && (dump || i == 0 || i == kMidXTensors - 1)) return hipErrorInvalidValue;
    for (int l = 0; l < kMidXLayers; ++l) {
      const MidXLayer& L = a.X[l];
      // one group of 32 channels; paired taps only for a first segment of
      // one word; a concat only in dec2.c1
      if (!L.w || L.cout <= 0 || L.cout > 32 || L.cw0 < 1 || (L.pair && L.cw0 != 1) || (L.cw1 != 0) != (l == 2))
        return hipErrorInvalidValue;
      if (dump && (!L.P || (l == 1 && !L.P2))) return hipErrorInvalidValue;
    }
    // the tensors' widths as the layers read them
    if (a.X[0].cw0 != a.xcw[0] || a.X[1].cw0 != a.xcw[1] || a.X[2].cw0 != a.xcw[2] || a.X[2].cw1 != a.cw[12] ||
        a.X[3].cw0 != a.xcw[3] || a.cw[0] != a.xcw[2] || a.dim[0] != 8 || a.dim[12] != 8)
      return hipErrorInvalidValue;
  }
  const size_t lds = (size_t)a.ldsw * 4;
  if (lds > 65536) return hipErrorInvalidValue;
  if (ext) {
    if (dump) hipLaunchKernelGGL((k_mid<true, true>), dim3(a.N), dim3(256), lds, s, a);
    else hipLaunchKernelGGL((k_mid<false, true>), dim3(a.N), dim3(256), lds, s, a);
  } else {
    if (dump) hipLaunchKernelGGL((k_mid<true, false>), dim3(a.N), dim3(256), lds, s, a);
    else hipLaunchKernelGGL((k_mid<false, false>), dim3(a.N), dim3(256), lds, s, a);
  }
  return hipGetLastError();
}

}  // namespace bnn
