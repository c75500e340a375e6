// bnn_bconv_mfma.hip - the v1 binary 3x3 conv on the int8 matrix cores of
// gfx950, with the rule (fold) and the fused 2x2 max-pool epilogues; layers
// with cout % 64 == 0.  Same P, bits and dumps as the popcount kernel
// (csrc/bnn_conv.c:23-36, csrc/bnn_maxpool.c:28-48).
//
// Built with the matrix instructions' accumulators in ordinary VGPRs
// (-mllvm -amdgpu-mfma-vgpr-form): with AGPR accumulators the compiler
// copies the 64 accumulator registers through VGPRs on every K step.
#include <algorithm>
#include <atomic>

#include "bnn_device.h"
#include "bnn_kernels.h"

namespace bnn {
namespace {

// ------------------------------------------------------------------------
// binary conv on the int8 matrix cores (cout % 64 == 0, fold / pool epilogues)
// ------------------------------------------------------------------------
// A block of four waves computes D for 64 output channels (4 groups of 16,
// the A operand: int8 +-1 weights) x one tile of 256 output pixels (each
// wave 4 groups of 16, the B operand: activation bits as 0/1 bytes) with
// v_mfma_i32_16x16x64_i8; P = 2*D - S[border class][co] (bnn_kernels.h).
// A tile is TR rows of TW columns of one patch (a patch of TR rows or more)
// or TI whole patches (smaller patches), TR * TW = 256: TW = W for rows up
// to 64 wide (whole rows), 32 for wider ones (W a power of two).
//
// B comes from LDS: for each chunk of two activation words the block stages
// the tile's rows with a one-pixel halo, (TR + 2) x (W + 2) pixels per patch,
// zeros outside the patch (and where a concat's upsample does not reach), so
// every tap of every pixel is a fixed offset from the pixel and no tap needs
// a mask.  A pixel's 64 bytes sit in an 80-byte slot and a row's slots are
// padded to 128 bytes mod 256, so the 16 lanes of a group (16 pixels of one
// row) read distinct banks.  Two buffers: chunk c + 1 is expanded and stored
// while chunk c is consumed, and its words are loaded from HBM one chunk
// earlier.  A (the same for the block's four waves) goes through LDS too:
// each K step's 64 channels x 64 bytes are loaded once per block (16 bytes
// a thread, four steps ahead of their use and two ahead of their store;
// one step ahead of the store measured 1-3% slower) into a ring of three slots, one
// barrier per K step, and each wave reads the next step's A from its slot
// while the current step's matrix ops run.  (Read straight from the weight
// table by every wave, A was the layer's bottleneck: the four waves'
// identical 4 KB per K step through the vector L1 held the matrix cores
// near a fifth of their rate.)
//
// One K step (64) is one tap of one chunk: lane group q = lane / 16 takes
// word q / 2 of the chunk, channels 16 * (q % 2) .. +15 of it, in A and B
// alike.  D register r of lane l holds channel 4 * (l / 16) + r, pixel l % 16
// of its group.  Fold tiles number pixels row by row.  Pool tiles give a
// group pair (0, 1 or 2, 3) the two rows of 8 consecutive 2x2 blocks, group
// 2p the top row, so a block's four pixels are lanes j, j ^ 1 of both groups.
// The epilogues rebuild each pixel's words: every lane folds its four
// channels and two lane swaps (v_permlane16_swap, v_permlane32_swap) gather
// the 16-bit group; the block max is a max across the pair and one DPP step.
typedef int i32x4v __attribute__((ext_vector_type(4)));

// 16 activation bits -> 16 bytes of 0/1, bit k to byte k: n * 0x00204081 is
// the OR of four shifted copies of the nibble n (they do not overlap), and
// bits 0, 8, 16, 24 of it are n's bits 0..3
__device__ __forceinline__ i32x4v bits_to_bytes(uint32_t b16) {
  i32x4v r;
#pragma unroll
  for (int k = 0; k < 4; ++k) r[k] = (int)((((b16 >> (4 * k)) & 0xFu) * 0x00204081u) & 0x01010101u);
  return r;
}
// OR of v over the four lane groups of 16 (lanes l, l ^ 16, l ^ 32, l ^ 48)
__device__ __forceinline__ uint32_t or_groups(uint32_t v) {
  const auto a = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = a[0] | a[1];
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return b[0] | b[1];
}
// max of x over lanes l, l ^ 1
__device__ __forceinline__ int32_t max_pair(int32_t x) {
  return max(x, __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false));  // quad_perm [1, 0, 3, 2]
}

constexpr int kSlot = 80;     // LDS bytes per staged pixel
constexpr int kStageMax = 2;  // staged pixels per thread and chunk
// A ring: 3 slots of 64 channels x 80 bytes (64 of weights, 16 of padding,
// so a read's 16 lanes of one 16-byte column hit distinct banks)
constexpr int kArow = 80;
constexpr uint32_t kAslot = 64 * kArow;
constexpr uint32_t kAring = 3 * kAslot;

struct MfmaTile {
  int lw, ltr, lti;     // log2 of TW, of rows per patch in a tile (min(TR, H)), of patches per tile
  int lcw;              // log2 of tiles across a row (W / TW)
  int hpt;              // tiles per patch (H / TR * W / TW), 1 for multi-patch tiles
  int rs, ps;           // LDS bytes per staged row, per staged patch
  FastDiv dps, drow;    // staged pixels per patch, per row
  int ns;               // staged pixels per chunk buffer
  uint32_t ntiles;
  uint32_t wbytes;      // weight table bytes
  int npair, nc0, nch;  // pairs; chunks of the first segment, in total
};

template <int EPI, bool DUMP>
__global__ __launch_bounds__(256) void k_bconv_mfma(const BconvArgs a, const int8_t* __restrict__ wi8,
                                                   const int32_t* __restrict__ stab, const MfmaTile T,
                                                   uint32_t bytes0, uint32_t bytes1) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr uint32_t kFar = 0x80000000u;
  const int tid = threadIdx.x, lane = tid & 63, q = lane >> 4, j = lane & 15, wave = tid >> 6;
  const int ncot = a.cout >> 6;  // 64-channel groups
  const uint32_t nitems = T.ntiles * (uint32_t)ncot;
  const int coutp = a.cout;
  const int h = q & 1;
  const int W = a.W, H = a.H;
  // this lane's pixel in each of its four groups, within a tile: patch,
  // row, column (the same for every tile)
  int pi[4], py[4], px[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    int l;  // tile-local row-major pixel index
    if (EPI == EPI_POOL) {
      // block 8 * (group pair) + j / 2 of the wave's 16, row g % 2 of it
      const int blk = 16 * wave + 8 * (g >> 1) + (j >> 1);
      const int bx = blk & ((1 << (T.lw - 1)) - 1), br = blk >> (T.lw - 1);  // block row within the tile
      l = ((2 * br + (g & 1)) << T.lw) + 2 * bx + (j & 1);
    } else {
      l = 64 * wave + 16 * g + j;
    }
    px[g] = l & ((1 << T.lw) - 1);
    const int r = l >> T.lw;
    py[g] = r & ((1 << T.ltr) - 1);
    pi[g] = r >> T.ltr;
  }
  const int lq = (q >> 1) * 32 + h * 16;  // this lane's 16 bytes in a slot
  uint32_t lb[4];
#pragma unroll
  for (int g = 0; g < 4; ++g)
    lb[g] = (uint32_t)(pi[g] * T.ps + (py[g] + 1) * T.rs + (px[g] + 1) * kSlot + lq);
  const uint32_t bufb = (uint32_t)(T.ps << T.lti);  // bytes per buffer

  const __amdgpu_buffer_rsrc_t rw = make_rsrc(wi8, T.wbytes);
  const __amdgpu_buffer_rsrc_t r0 = make_rsrc(a.in0, bytes0);
  const __amdgpu_buffer_rsrc_t r1 = make_rsrc(a.in1 ? a.in1 : a.in0, bytes1);
  const uint32_t cw0b = (uint32_t)a.cw0 * 4u, cw1b = (uint32_t)a.cw1 * 4u;
  // item it: tile it / ncot (patches n0 .. n0 + 2^lti - 1, rows y0 ..
  // y0 + 2^ltr - 1
  // (columns x0 .. x0 + TW - 1), output channels 64 * (it % ncot) ..
  auto tile_n0 = [&](uint32_t it) { return (int)((it / (uint32_t)ncot) / (uint32_t)T.hpt) << T.lti; };
  auto tile_y0 = [&](uint32_t it) { return (int)(((it / (uint32_t)ncot) % (uint32_t)T.hpt) >> T.lcw) << T.ltr; };
  auto tile_x0 = [&](uint32_t it) {
    return (int)(((it / (uint32_t)ncot) % (uint32_t)T.hpt) & ((1u << T.lcw) - 1u)) << T.lw;
  };

  // ---- staging: the two words of chunk c of item it for this thread's staged pixels
  uint32_t sw[kStageMax][2];
  auto stage_load = [&](uint32_t it, int c) {
    const int n0 = tile_n0(it), y0 = tile_y0(it), x0 = tile_x0(it);
    const bool s1 = c >= T.nc0;
    const int wd = 2 * (s1 ? c - T.nc0 : c);
    const bool two = wd + 1 < (s1 ? a.cw1 : a.cw0);
#pragma unroll
    for (int k = 0; k < kStageMax; ++k) {
      const uint32_t i = (uint32_t)(tid + 256 * k);
      const uint32_t ip = fdiv(i, T.dps), ir = i - ip * T.dps.d, rr = fdiv(ir, T.drow), cc = ir - rr * T.drow.d;
      const int n = n0 + (int)ip, y = y0 + (int)rr - 1, x = x0 + (int)cc - 1;
      bool ok = i < (uint32_t)T.ns && n < a.N && (unsigned)y < (unsigned)H && (unsigned)x < (unsigned)W;
      uint32_t off;
      if (!s1) {
        off = (((uint32_t)n * (uint32_t)H + (uint32_t)y) * (uint32_t)W + (uint32_t)x) * cw0b + (uint32_t)wd * 4u;
      } else {
        // nearest 2x upsample placed at (oh, ow); positions it does not
        // cover read 0 bits
        const int uy = y - a.oh, ux = x - a.ow;
        ok = ok && (unsigned)uy < (unsigned)a.uh && (unsigned)ux < (unsigned)a.uw;
        off = (((uint32_t)n * (uint32_t)a.h1 + (uint32_t)(uy >> 1)) * (uint32_t)a.w1 + (uint32_t)(ux >> 1)) * cw1b +
              (uint32_t)wd * 4u;
      }
      off = ok ? off : kFar;
      sw[k][0] = ld_u32(s1 ? r1 : r0, off, 0);
      sw[k][1] = two ? ld_u32(s1 ? r1 : r0, off + 4u, 0) : 0u;
    }
  };
  auto stage_store = [&](int buf) {
#pragma unroll
    for (int k = 0; k < kStageMax; ++k) {
      const uint32_t i = (uint32_t)(tid + 256 * k);
      if (i < (uint32_t)T.ns) {
        const uint32_t ip = fdiv(i, T.dps), ir = i - ip * T.dps.d, rr = fdiv(ir, T.drow), cc = ir - rr * T.drow.d;
        uint8_t* d = smem + (uint32_t)buf * bufb + ip * (uint32_t)T.ps + rr * (uint32_t)T.rs + cc * kSlot;
#pragma unroll
        for (int w2 = 0; w2 < 2; ++w2)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh)
            *reinterpret_cast<i32x4v*>(d + 32 * w2 + 16 * hh) = bits_to_bytes((sw[k][w2] >> (16 * hh)) & 0xFFFFu);
      }
    }
  };

  // ---- A: each thread stages 16 bytes of a K step's 64 x 64 weight
  // bytes: channel ac = tid / 4 of the item's group, bytes 16 * (tid % 4);
  // the table row of channel co, K step st is 64 bytes at (co * npair + 2 st) * 32
  const int ac = tid >> 2, ap = tid & 3;
  auto a_piece = [&](uint32_t itm, int st) {
    return (uint32_t)((((int)(itm % (uint32_t)ncot) * 64 + ac) * T.npair + 2 * st) * 32 + 16 * ap);
  };
  auto a_load = [&](uint32_t itm, int st) {
    return __builtin_bit_cast(i32x4v, __builtin_amdgcn_raw_buffer_load_b128(rw, (int)a_piece(itm, st), 0, 0));
  };
  const uint32_t aring = 2 * bufb;  // the ring after the two staging buffers
  auto a_store = [&](uint32_t slot, const i32x4v& v) {
    *reinterpret_cast<i32x4v*>(smem + aring + slot * kAslot + (uint32_t)(ac * kArow + 16 * ap)) = v;
  };
  // the wave's operand A[m] (channel 16 m + j, K bytes 16 q ..) from a slot
  auto a_read = [&](uint32_t slot, i32x4v (&A)[4]) {
#pragma unroll
    for (int m = 0; m < 4; ++m)
      A[m] = *reinterpret_cast<const i32x4v*>(smem + aring + slot * kAslot + (uint32_t)((16 * m + j) * kArow + 16 * q));
  };

  i32x4v acc[4][4];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int g = 0; g < 4; ++g) acc[m][g] = i32x4v{0, 0, 0, 0};

  // This block's items, XCD-aware: blocks go to the XCDs in turn (block b
  // to XCD b % 8, the grid a multiple of 8), XCD x takes the tiles
  // x, x + 8, x + 16, ... and its blocks walk that list's items (tile, then
  // channel group fastest) in turn, so a tile's channel groups, which read
  // the same staged rows and write different words of the same pixels, run
  // side by side on one XCD and their stores merge in its L2.  Local item
  // li of XCD x is tile (li / ncot) * 8 + x, group li % ncot; the chunks of
  // all of a block's items form one pipeline.
  const uint32_t xcd = blockIdx.x & 7u, nslot = gridDim.x >> 3;
  auto item_of = [&](uint32_t li) -> uint32_t {
    const uint32_t tile = (li / (uint32_t)ncot) * 8u + xcd;
    return tile < T.ntiles ? tile * (uint32_t)ncot + li % (uint32_t)ncot : 0xFFFFFFFFu;
  };
  uint32_t li = blockIdx.x >> 3;
  uint32_t it = item_of(li);
  if (it >= nitems) return;
  stage_load(it, 0);
  stage_store(0);
  // the chunk after (it, c) is (it, c + 1), or (the block's next item, 0)
  uint32_t lli = li, lit = it;  // item and chunk of the staged-ahead words in sw
  int lc = 0;
  bool lok = true;
  auto advance = [&]() {
    if (++lc == T.nch) {
      lc = 0;
      lli += nslot;
      lit = item_of(lli);
      lok = lit < nitems;
    }
  };
  advance();
  if (lok) stage_load(lit, lc);
  // the K steps of the block's items run as one sequence: step S (item
  // steps st = c * 9 + t) takes A from slot S % 3; at its start (a barrier)
  // A of step S + 1 is visible and slot (S + 2) % 3 is free
  const int nst = T.nch * 9;  // K steps per item
  auto a_load_ahead = [&](int st) {  // A of in-item step st, or of the next item past its end
    return st < nst ? a_load(it, st) : a_load(item_of(li + nslot), st - nst);
  };
  a_store(0, a_load(it, 0));
  a_store(1, a_load_ahead(1));
  i32x4v ag = a_load_ahead(2);   // A of step S + 2, stored during step S
  i32x4v ag2 = a_load_ahead(3);  // A of step S + 3
  __syncthreads();
  i32x4v Ar[4];
  a_read(0, Ar);
  uint32_t S = 0;
  int buf = 0;
#pragma unroll 1
  for (;;) {
#pragma unroll 1
    for (int c = 0; c < T.nch; ++c) {
      const uint32_t bo = (uint32_t)buf * bufb;
#pragma unroll
      for (int t = 0; t < 9; ++t) {
        const int ky = t / 3, kx = t % 3;
        __syncthreads();
        const uint32_t s0 = S % 3u, s1 = s0 == 2u ? 0u : s0 + 1u, s2 = s1 == 2u ? 0u : s1 + 1u;
        i32x4v An[4];
        a_read(s1, An);
        const uint32_t dt = bo + (uint32_t)((ky - 1) * T.rs + (kx - 1) * kSlot);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const i32x4v B = *reinterpret_cast<const i32x4v*>(smem + lb[g] + dt);
#pragma unroll
          for (int m = 0; m < 4; ++m) acc[m][g] = __builtin_amdgcn_mfma_i32_16x16x64_i8(Ar[m], B, acc[m][g], 0, 0, 0);
        }
        // A of step S + 2 into its slot, the load of step S + 4
        a_store(s2, ag);
        ag = ag2;
        ag2 = a_load_ahead(c * 9 + t + 4);
#pragma unroll
        for (int m = 0; m < 4; ++m) Ar[m] = An[m];
        ++S;
      }
      // the next chunk into the other buffer (visible after the next step's
      // barrier), the one after it from HBM
      if (lok) {
        stage_store(buf ^ 1);
        advance();
        if (lok) stage_load(lit, lc);
      }
      buf ^= 1;
    }
    // ---------------------------------------------------------- epilogue --
    // one group of 16 channels at a time: P, the rule, and the gather into
    // 16-bit halves of the output words; then the word stores
    {
      const int n0 = tile_n0(it), y0 = tile_y0(it), x0 = tile_x0(it);
      const int co0 = (int)(it % (uint32_t)ncot) * 64;
      const int HW = H * W;
      const int Hh = H >> 1, Wh = W >> 1;
      int cls[4];
      bool pv[4];
      size_t pix[4];  // global pixel index
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int y = y0 + py[g], x = x0 + px[g];
        pv[g] = n0 + pi[g] < a.N;
        cls[g] = ((y == 0 ? 1 : 0) | (y == H - 1 ? 2 : 0)) * 4 + ((x == 0 ? 1 : 0) | (x == W - 1 ? 2 : 0));
        pix[g] = ((size_t)(n0 + pi[g]) * H + y) * W + x;
      }
      uint32_t half[4][4], half2[4][2];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int cb = co0 + 16 * m + 4 * q;  // this lane's four channels cb .. cb+3
        const i32x4v lo1 = *reinterpret_cast<const i32x4v*>(a.f1.lo + cb);
        const i32x4v wd1 = *reinterpret_cast<const i32x4v*>(a.f1.wid + cb);
        int32_t P[4][4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const i32x4v sv = *reinterpret_cast<const i32x4v*>(stab + (size_t)cls[g] * coutp + cb);
          uint32_t nib = 0;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            P[g][r] = 2 * acc[m][g][r] - sv[r];
            nib |= ((uint32_t)P[g][r] - (uint32_t)lo1[r] < (uint32_t)wd1[r] ? 1u : 0u) << r;
            if (DUMP && pv[g]) a.P[((size_t)(n0 + pi[g]) * a.cout + cb + r) * HW + (size_t)(y0 + py[g]) * W + x0 + px[g]] = P[g][r];
          }
          half[m][g] = or_groups(nib << (4 * q));
        }
        if constexpr (EPI == EPI_POOL) {
          const i32x4v lo2 = *reinterpret_cast<const i32x4v*>(a.f2.lo + cb);
          const i32x4v wd2 = *reinterpret_cast<const i32x4v*>(a.f2.wid + cb);
#pragma unroll
          for (int p = 0; p < 2; ++p) {
            uint32_t nib2 = 0;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int32_t pm = max_pair(max(P[2 * p][r], P[2 * p + 1][r]));
              nib2 |= ((uint32_t)pm - (uint32_t)lo2[r] < (uint32_t)wd2[r] ? 1u : 0u) << r;
              if (DUMP && pv[2 * p] && (j & 1) == 0)
                a.P2[((size_t)(n0 + pi[2 * p]) * a.cout + cb + r) * Hh * Wh + (size_t)((y0 + py[2 * p]) >> 1) * Wh +
                     ((x0 + px[2 * p]) >> 1)] = pm;
            }
            half2[m][p] = or_groups(nib2 << (4 * q));
          }
        }
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        if (a.out != nullptr && pv[g] && q < 2) {  // a pooled layer may skip its full-size bits
          const uint32_t word = q == 0 ? (half[0][g] | half[1][g] << 16) : (half[2][g] | half[3][g] << 16);
          a.out[pix[g] * a.cwo + (co0 >> 5) + q] = word;
        }
      }
      if constexpr (EPI == EPI_POOL) {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          if (pv[2 * p] && (j & 1) == 0 && q < 2) {
            const uint32_t word = q == 0 ? (half2[0][p] | half2[1][p] << 16) : (half2[2][p] | half2[3][p] << 16);
            const size_t dp = ((size_t)(n0 + pi[2 * p]) * Hh + ((y0 + py[2 * p]) >> 1)) * Wh + ((x0 + px[2 * p]) >> 1);
            a.out2[dp * a.cwo + (co0 >> 5) + q] = word;
          }
        }
      }
    }
    li += nslot;
    it = item_of(li);
    if (it >= nitems) break;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int g = 0; g < 4; ++g) acc[m][g] = i32x4v{0, 0, 0, 0};
  }
}

}  // namespace

// The tile of a (H, W) layer: TR = 256 / TW rows of TW columns of a patch
// (TW = W up to 64 wide, else 32), or 256 / (H W) whole patches; false when
// the shape has no such tile or its two staging buffers exceed 64 KB of LDS
// (with the A ring, under 80 KB: two blocks a CU).
static bool mfma_tile(int H, int W, int epi, MfmaTile* T) {
  if (W < 8 || (W & (W - 1)) || W > (1 << 20) || H <= 0) return false;
  if (epi == EPI_POOL && (H & 1)) return false;
  const int TW = W > 64 ? 32 : W;
  const int TR = 256 / TW;
  int ltr = 0, lti = 0, hpt = 1, lcw = 0;
  while ((TW << lcw) < W) ++lcw;
  if (H >= TR) {
    if (H % TR) return false;
    hpt = (H / TR) << lcw;
    while ((1 << ltr) < TR) ++ltr;
  } else {
    if (TW != W || TR % H || (H & (H - 1))) return false;
    while ((1 << ltr) < H) ++ltr;
    while ((1 << lti) < TR / H) ++lti;
  }
  int lw = 0;
  while ((1 << lw) < TW) ++lw;
  const int rows = (1 << ltr) + 2, cols = TW + 2;
  int rs = cols * kSlot;
  rs += (128 - rs % 256 + 256) % 256;  // rows 128 bytes apart mod 256
  int ps = rows * rs;
  if (2 * (ps << lti) > 65536) {  // no room for the padding
    rs = cols * kSlot;
    ps = rows * rs;
  }
  if (2 * (ps << lti) > 65536) return false;
  const int ns = (rows * cols) << lti;
  if (ns > 256 * kStageMax) return false;
  if (T) {
    T->lw = lw; T->ltr = ltr; T->lti = lti; T->lcw = lcw; T->hpt = hpt;
    T->rs = rs; T->ps = ps;
    T->dps = make_fastdiv((uint32_t)(rows * cols));
    T->drow = make_fastdiv((uint32_t)cols);
    T->ns = ns;
  }
  return true;
}

bool mfma_conv_fits(int cout, int H, int W, int epi) {
  return cout % 64 == 0 && (epi == EPI_FOLD || epi == EPI_POOL) && mfma_tile(H, W, epi, nullptr);
}

hipError_t launch_bconv_mfma(const BconvArgs& a, const MfmaConv& mc, int epi, bool dump, hipStream_t s) {
  if (a.N <= 0 || a.H <= 0 || a.W <= 0) return hipSuccess;
  MfmaTile T{};
  if ((epi != EPI_FOLD && epi != EPI_POOL) || !mc.w || !mc.s || a.cout % 64 || !mfma_tile(a.H, a.W, epi, &T))
    return hipErrorInvalidValue;
  if (a.in1 && a.padoff != 0x80000000u) return hipErrorInvalidValue;  // v1 concat semantics only
  if (dump && (!a.P || (epi == EPI_POOL && !a.P2))) return hipErrorInvalidValue;  // dumps need their targets
  const size_t npix = (size_t)a.N * a.H * a.W;
  if (npix * a.cw0 * 4 >= 0x80000000ull) return hipErrorInvalidValue;
  if (a.in1 && (size_t)a.N * a.h1 * a.w1 * a.cw1 * 4 >= 0x80000000ull) return hipErrorInvalidValue;
  T.npair = mc.npair;
  T.nc0 = (a.cw0 + 1) / 2;
  T.nch = mfma_nchunk(a.cw0, a.in1 ? a.cw1 : 0);
  if (T.npair != 18 * T.nch) return hipErrorInvalidValue;
  const size_t wbytes = (size_t)a.cout * T.npair * 32;
  if (wbytes + 64 * 32 >= 0x80000000ull) return hipErrorInvalidValue;
  T.wbytes = (uint32_t)wbytes;
  const size_t per = (size_t)1 << T.lti;  // patches per tile
  const size_t ntiles = T.lti ? (a.N + per - 1) / per : (size_t)a.N * T.hpt;
  if (ntiles >= 0x7FFFFFFFull) return hipErrorInvalidValue;
  T.ntiles = (uint32_t)ntiles;
  const uint32_t b0 = (uint32_t)(npix * a.cw0 * 4);
  const uint32_t b1 = a.in1 ? (uint32_t)((size_t)a.N * a.h1 * a.w1 * a.cw1 * 4) : 0u;
  const size_t lds = (size_t)2 * ((size_t)T.ps << T.lti) + kAring;
  // more than 64 KB of LDS: allowed once per variant and device (bit d of
  // the variant's mask for device d)
  using Fn = void (*)(const BconvArgs, const int8_t*, const int32_t*, const MfmaTile, uint32_t, uint32_t);
  static const Fn fns[4] = {k_bconv_mfma<EPI_FOLD, false>, k_bconv_mfma<EPI_FOLD, true>, k_bconv_mfma<EPI_POOL, false>,
                            k_bconv_mfma<EPI_POOL, true>};
  static std::atomic<uint64_t> attr[4];
  const int var = (epi == EPI_POOL ? 2 : 0) + (dump ? 1 : 0);
  // as many blocks as fit on the chip at once (LDS, and three waves per
  // SIMD by registers), each walking items blockIdx.x, + gridDim.x, ...
  int dev = 0, cus = 0;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  const uint64_t bit = 1ull << (dev & 63);
  if (!(attr[var].load(std::memory_order_acquire) & bit)) {
    if (hipError_t e = hipFuncSetAttribute((const void*)fns[var], hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        e != hipSuccess)
      return e;
    attr[var].fetch_or(bit, std::memory_order_acq_rel);
  }
  const size_t per_cu = std::min<size_t>(3, (160 * 1024) / lds);
  const size_t items = ntiles * (size_t)(a.cout / 64);
  if (items >= 0xFFFFFFFFull) return hipErrorInvalidValue;
  // (a multiple of 8 blocks for the XCD-aware item order; blocks without
  // an item exit)
  const dim3 grid((unsigned)((std::min<size_t>(items, per_cu * cus) + 7) / 8 * 8));
  hipLaunchKernelGGL(fns[var], grid, dim3(256), lds, s, a, mc.w, mc.s, T, b0, b1);
  return hipGetLastError();
}

}  // namespace bnn
