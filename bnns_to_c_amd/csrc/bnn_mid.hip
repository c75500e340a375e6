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

template <bool DUMP>
__global__ __launch_bounds__(256) void k_mid(const MidArgs a) {
  extern __shared__ uint32_t mlds[];
  const int n = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  MidT T[kMidTensors];
#pragma unroll
  for (int i = 0; i < kMidTensors; ++i) T[i] = MidT{a.off[i], a.dim[i], a.cw[i]};
  // the input (enc2's pooled bits, 8 x 8, [pixel][word] in memory) into
  // LDS, planar by word
  {
    const int cw = T[0].cw, nw = 64 * cw;
    const uint32_t* src = a.t[0] + (size_t)n * nw;
    for (int k = tid; k < nw; k += 256) {
      const int w = k >> 6, p = k & 63;
      mlds[T[0].off + k] = src[p * cw + w];
    }
  }
  __syncthreads();
  const MidT none{0, 0, 0};
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
  // out: dec3.c2's bits; the debug forward also takes every intermediate
#pragma unroll 1
  for (int i = DUMP ? 1 : kMidTensors - 1; i < kMidTensors; ++i) {
    const int cw = T[i].cw, np = T[i].d * T[i].d, nw = np * cw;
    uint32_t* dst = a.t[i] + (size_t)n * nw;
    for (int k = tid; k < nw; k += 256) {
      const int p = k / cw, w = k - p * cw;
      dst[k] = mlds[T[i].off + w * np + p];
    }
  }
}

}  // namespace

hipError_t launch_mid(const MidArgs& a, bool dump, hipStream_t s) {
  if (a.N <= 0) return hipSuccess;
  for (int i = 0; i < kMidTensors; ++i) {
    if (!a.t[i] && (dump || i == 0 || i == kMidTensors - 1)) return hipErrorInvalidValue;
    // 128-bit row reads: every tensor starts on 4 words
    if (a.off[i] % 4) return hipErrorInvalidValue;
  }
  if (dump)
    for (int l = 0; l < kMidLayers; ++l)
      if (!a.L[l].P || ((l == 1 || l == 3) && !a.L[l].P2)) return hipErrorInvalidValue;
  const size_t lds = (size_t)a.ldsw * 4;
  if (lds > 65536) return hipErrorInvalidValue;
  if (dump) hipLaunchKernelGGL(k_mid<true>, dim3(a.N), dim3(256), lds, s, a);
  else hipLaunchKernelGGL(k_mid<false>, dim3(a.N), dim3(256), lds, s, a);
  return hipGetLastError();
}

}  // namespace bnn
