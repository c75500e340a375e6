// bnn_kernels.hip - gfx950 kernels for the v1 Bi-Real binary UNet forward.
//
// Binary conv (csrc/bnn_conv.c:23-36): per output pixel and channel
//     P = sum over in-image taps of a*w = N_valid - 2 * popcount((a XOR w) & valid)
// with N_valid = (#in-image taps) * Cin.  Activations and weights are packed
// along channels (bit = sign > 0), so each 32-bit word of a tap costs one
// v_bitop3_b32 ((a ^ w) & valid) and one v_bcnt_u32_b32 (popcount + acc).
// Zero high bits in both operands contribute nothing, so channel tails and
// the word-aligned [skip ; upsampled] concat need no extra masking.  A work
// item is one output pixel (MT=1) or a 2x2 block (MT=2, used by the pool
// epilogue); the COG output channels of its group are wave-uniform, so the
// weights arrive through scalar loads and feed the VALU as SGPR operands.
// P never leaves registers: the integer rule, the 2x2 max-pool, the second
// rule and the fp32 head run in the epilogue.
//
// Real-input first conv (csrc/bnn_conv_realin.c:66-116) is order-exact: for
// each output, taps in row-major order, s = x*w summed over ci from 0 in
// sequence, acc += s, out = alpha * acc.  Every product is x * (+-1), which
// is exact, so one fused multiply-add per term rounds exactly like the
// reference's multiply-then-add.  Out-of-image taps read zeros and sum to
// +0; skipping a tap and adding that +0 are the same, since s and acc never
// hold -0.
#include <algorithm>
#include <utility>

#include "bnn_device.h"
#include "bnn_kernels.h"

// Multi-dword raw buffer loads, declared on the LLVM intrinsics themselves:
// clang's __builtin_amdgcn_raw_buffer_load_b64 / _b128 keep only the first
// dword on this toolchain (the other elements of the result repeat it).
typedef float stem_f32x2 __attribute__((ext_vector_type(2)));
typedef float stem_f32x4 __attribute__((ext_vector_type(4)));
extern "C" __device__ stem_f32x2 raw_load_f32x2(__amdgpu_buffer_rsrc_t rsrc, int voffset, int soffset, int aux) __asm(
    "llvm.amdgcn.raw.ptr.buffer.load.v2f32");
extern "C" __device__ stem_f32x4 raw_load_f32x4(__amdgpu_buffer_rsrc_t rsrc, int voffset, int soffset, int aux) __asm(
    "llvm.amdgcn.raw.ptr.buffer.load.v4f32");
extern "C" __device__ void raw_store_f32x2(stem_f32x2 vdata, __amdgpu_buffer_rsrc_t rsrc, int voffset, int soffset,
                                           int aux) __asm("llvm.amdgcn.raw.ptr.buffer.store.v2f32");

namespace bnn {
namespace {

constexpr int kBlock = 256;


// ------------------------------------------------------------------------
// real-input conv + real fold
// ------------------------------------------------------------------------
// Work-group: an RT x RW output tile for RG groups of RCO output channels.
// Each lane of a group owns PXR vertically adjacent pixels of one column;
// the RT x RW tile takes RT/PXR x RW lanes per group (whole waves).  The
// (RT+2) x (RW+2) input tile, CI channels at a time, is staged in LDS,
// double-buffered, with zeros outside the image (buffer loads out of range
// return 0), and shared by all groups, so each input byte is fetched once per
// tile.  Each lane keeps the 9 per-tap in-order sums of its RCO channels for
// each of its pixels over all ci, then adds them into acc in row-major tap
// order; an out-of-image tap sums zeros to +0, which leaves acc unchanged.
// Every weight fetched through the scalar path feeds PXR FMAs.
#ifndef BNN_RCI
#define BNN_RCI 8
#endif
constexpr int RT = 8, RW = 32, RCO = BNN_RCO, PXR = BNN_PXR, CI = BNN_RCI;
constexpr int LR = RT + 2, LC = RW + 2, LTILE = CI * LR * LC;
constexpr int RLANES = RT / PXR * RW;  // lanes per channel group

template <int RG>
__global__ __launch_bounds__(RLANES * RG) void k_real_conv(const RealArgs a, uint32_t xbytes, int tilesH,
                                                           int tilesW) {
  static_assert(RLANES % 64 == 0, "channel groups must be whole waves");
  static_assert(32 % RCO == 0, "a channel group must not straddle a 32-bit word");
  constexpr int NT = RLANES * RG;
  constexpr int KL = (LTILE + NT - 1) / NT;
  constexpr int OW = (RG * RCO + 31) / 32;  // output words per pixel this block writes
  __shared__ float tile[2][LTILE];
  __shared__ uint32_t obits[RT * RW * OW];
  const int tid = threadIdx.x;
  for (int i = tid; i < RT * RW * OW; i += NT) obits[i] = 0;
  // a group is a whole number of waves: the group index is wave-uniform
  const int grp = __builtin_amdgcn_readfirstlane(tid / RLANES);
  const int lt = tid - grp * RLANES;
  const int r0 = (lt / RW) * PXR, c = lt % RW;
  int bid = blockIdx.x;
  const int tx = bid % tilesW;
  bid /= tilesW;
  const int ty = bid % tilesH;
  const int n = bid / tilesH;
  const int y0 = ty * RT, x0 = tx * RW;
  const int cog = blockIdx.y * RG + grp;  // global channel group
  const int HW = a.H * a.W;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.x, xbytes);

  // this thread's share of every chunk load: byte offset within the chunk,
  // or an offset past the buffer (reads 0) for positions outside the image,
  // and where it goes in the [row][ci][col] tile (all CI channels and 3
  // columns of a tile row lie within one ds_read2 offset range)
  const InGeom ig = in_geom(a, n);
  uint32_t goff[KL];
  int lidx[KL];
#pragma unroll
  for (int k = 0; k < KL; ++k) {
    const int e = tid + k * NT;
    const int cil = e / (LR * LC), rem = e - cil * (LR * LC);
    const int row = rem / LC, col = rem - row * LC;
    lidx[k] = e < LTILE ? (row * CI + cil) * LC + col : 0;
    const int gy = y0 - 1 + row, gx = x0 - 1 + col;
    const bool ok = e < LTILE && gy >= 0 && gy < ig.ylim && gx >= 0 && gx < ig.xlim;
    goff[k] = ok ? (uint32_t)(ig.base + cil * ig.cstride + (size_t)gy * ig.rstride + gx) * 4u : 0x80000000u;
  }
  const uint32_t chunk_bytes = (uint32_t)(CI * ig.cstride * 4u);
  const int nchunk = (a.cin + CI - 1) / CI;

  float st[PXR][9][RCO];
#pragma unroll
  for (int p = 0; p < PXR; ++p)
#pragma unroll
    for (int t = 0; t < 9; ++t)
#pragma unroll
      for (int g = 0; g < RCO; ++g) st[p][t][g] = 0.0f;

  float pre[KL];
#pragma unroll
  for (int k = 0; k < KL; ++k) pre[k] = ld_f32(rs, goff[k], 0);
#pragma unroll
  for (int k = 0; k < KL; ++k)
    if (tid + k * NT < LTILE) tile[0][lidx[k]] = pre[k];
  __syncthreads();

  const float* wg = a.w + (size_t)cog * a.cin * 9 * RCO;  // [cin][9][RCO] of this group
  const int lbase = r0 * CI * LC + c;
#pragma unroll 1
  for (int ch = 0; ch < nchunk; ++ch) {
    const int buf = ch & 1;
    const bool more = ch + 1 < nchunk;
    if (more) {
#pragma unroll
      for (int k = 0; k < KL; ++k) pre[k] = ld_f32(rs, goff[k], (uint32_t)(ch + 1) * chunk_bytes);
    }
    const int ci0 = ch * CI;
    const int nci = a.cin - ci0 < CI ? a.cin - ci0 : CI;
    const float* tb = tile[buf] + lbase;
#pragma unroll
    for (int cl = 0; cl < CI; ++cl) {
      if (cl < nci) {
        float xv[PXR + 2][3];
#pragma unroll
        for (int i = 0; i < PXR + 2; ++i)
#pragma unroll
          for (int kx = 0; kx < 3; ++kx) xv[i][kx] = tb[(i * CI + cl) * LC + kx];
        const float* wp = wg + (size_t)(ci0 + cl) * 9 * RCO;
#pragma unroll
        for (int t = 0; t < 9; ++t)
#pragma unroll
          for (int g = 0; g < RCO; ++g) {
            const float w = wp[t * RCO + g];
#pragma unroll
            for (int p = 0; p < PXR; ++p) st[p][t][g] = __fmaf_rn(xv[p + t / 3][t % 3], w, st[p][t][g]);
          }
      }
    }
    if (more) {
#pragma unroll
      for (int k = 0; k < KL; ++k)
        if (tid + k * NT < LTILE) tile[buf ^ 1][lidx[k]] = pre[k];
    }
    __syncthreads();
  }

  const int co0 = cog * RCO;
  const int nco = a.cout - co0 < RCO ? a.cout - co0 : RCO;
  const int cwo = (a.cout + 31) >> 5;
  const int cb0 = blockIdx.y * RG * RCO;  // first channel of this block (a multiple of 32 when gridDim.y > 1)
#pragma unroll
  for (int p = 0; p < PXR; ++p) {
    float acc[RCO];
#pragma unroll
    for (int g = 0; g < RCO; ++g) acc[g] = 0.0f;
#pragma unroll
    for (int t = 0; t < 9; ++t)
#pragma unroll
      for (int g = 0; g < RCO; ++g) acc[g] = __fadd_rn(acc[g], st[p][t][g]);
    const int y = y0 + r0 + p, x = x0 + c;
    if (y >= a.H || x >= a.W || co0 >= a.cout) continue;
    if (a.f32) {
#pragma unroll
      for (int g = 0; g < RCO; ++g)
        if (g < nco)
          a.f32[((size_t)n * a.cout + co0 + g) * HW + (size_t)y * a.W + x] = __fmul_rn(a.alpha[co0 + g], acc[g]);
    }
    if (a.out) {
      // real fold (csrc/bnn_fold.c:62-77): z = fma(A, x, B); z<0 -> slope*z;
      // r = z + rsign; bit = r > 0.  The reference build fuses A*x+B only.
      uint32_t bits = 0;
#pragma unroll
      for (int g = 0; g < RCO; ++g) {
        const int co = co0 + g;
        const float o = __fmul_rn(a.alpha[co], acc[g]);
        float z = __fmaf_rn(a.A[co], o, a.B[co]);
        if (z < 0.0f) z = __fmul_rn(a.slope[co], z);
        const float rr = __fadd_rn(z, a.rsign[co]);
        bits |= (rr > 0.0f && g < nco) ? (1u << g) : 0u;
      }
      const int cl = co0 - cb0;  // RCO divides 32: a group never straddles a word
      atomicOr(&obits[((r0 + p) * RW + c) * OW + (cl >> 5)], bits << (cl & 31));
    }
  }
  if (!a.out) return;
  // whole words of the block's channels (bits above cout stay 0)
  __syncthreads();
  for (int i = tid; i < RT * RW * OW; i += NT) {
    const int pl = i / OW, wd = i - pl * OW;
    const int y = y0 + pl / RW, x = x0 + pl % RW;
    const int word = (cb0 >> 5) + wd;
    if (y < a.H && x < a.W && word < cwo)
      a.out[((size_t)n * HW + (size_t)y * a.W + x) * cwo + word] = obits[i];
  }
}

// ------------------------------------------------------------------------
// real-input conv on the matrix cores
// ------------------------------------------------------------------------
// v_mfma_f32_16x16x1_4b_f32 computes, for 4 blocks b, D_b[i][j] =
// fma(A[i], B_b[j], C_b[i][j]), each element rounded once to nearest even:
// with K = 1 an element is exactly one step s = fma(x, w, s) of the
// reference's per-tap chain (the device matches fmaf bit for bit, signed
// zeros and denormals included).  Rows i are 16 output channels, columns j
// 16 pixels of an output row, blocks 4 consecutive rows, so a wave owns a
// 4 x 16 pixel tile and keeps one 16-register accumulator block per tap.
// Operand B is the input value the lane's pixel sees through the tap, read
// from the LDS tile.  Operand A is the +-1 weight of row i: with CBSZ = 2 the
// A values of block ABID feed all four blocks, so one register holds the
// weights of four taps (lanes 16k..16k+15 = tap 4q+k), made from a lane mask
// by one v_cndmask.  Lane layout: B lane l -> block l/16, column l%16;
// D register r of lane l -> block r/4, row 4*(l/16) + r%4, column l%16.
typedef float f32x16 __attribute__((ext_vector_type(16)));

// the nine taps of one input channel: tap t takes A from block t%4 of
// register wa[t/4] (the broadcast fields must be literal constants)
template <int T>
__device__ __forceinline__ void mfma_tap(f32x16 (&acc)[9], const float (&wa)[3], const float (&xb)[9]) {
  acc[T] = __builtin_amdgcn_mfma_f32_16x16x1f32(wa[T >> 2], xb[T], acc[T], 2, T & 3, 0);
}
template <int... T>
__device__ __forceinline__ void mfma_taps(f32x16 (&acc)[9], const float (&wa)[3], const float (&xb)[9],
                                          std::integer_sequence<int, T...>) {
  (mfma_tap<T>(acc, wa, xb), ...);
}
// v3 order: the nine taps of one input channel as consecutive steps of one
// chain (csrc/bnn_realin_blk.h:111-125)
template <int T>
__device__ __forceinline__ void mfma_chain_tap(f32x16& acc, const float (&wa)[3], const float (&xb)[9]) {
  acc = __builtin_amdgcn_mfma_f32_16x16x1f32(wa[T >> 2], xb[T], acc, 2, T & 3, 0);
}
template <int... T>
__device__ __forceinline__ void mfma_chain(f32x16& acc, const float (&wa)[3], const float (&xb)[9],
                                           std::integer_sequence<int, T...>) {
  (mfma_chain_tap<T>(acc, wa, xb), ...);
}

#ifndef BNN_MWPE
#define BNN_MWPE 2
#endif
#ifndef BNN_MWPE_RX
#define BNN_MWPE_RX 3
#endif
#ifndef BNN_MLC_RX
#define BNN_MLC_RX 48
#endif
#ifndef BNN_MLC
#define BNN_MLC 80
#endif
// an offset past any input of the matrix-core real conv (inputs are smaller)
constexpr uint32_t kRealFar = 0x7FFFFFF0u;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// waves along rows / columns: tile (4*WR) x (16*WC); PARTIAL: cin is not a
// multiple of the chunk size.  RX: the v3 (ReActNet) enc1 unit 1 -- one
// conv chain per output over ci outermost and taps inside
// (csrc/bnn_realin_blk.h:111-125), a 1x1 projection chain on the centre tap
// with real weights (csrc/bnn_realin_blk.h:59-70), and the epilogue
// h = RPReLU(fma(A, alpha*acc, B + move1) + proj) written as float planes
// with the bits of the next tap on h (csrc/bnn_react_epi.c:57-77,
// bnn_react_ops.c:75-85).  The projection weights of a chunk ride along
// with its input rows: one more LDS-writing load per wave.
template <int WR, int WC, bool PARTIAL, bool RX>
__global__ __launch_bounds__(64 * WR * WC) __attribute__((amdgpu_waves_per_eu(RX ? BNN_MWPE_RX : BNN_MWPE)))
void k_real_mfma(const RealArgs a, uint32_t xbytes, int tilesH, int tilesW) {
  constexpr int TR = 4 * WR, TC = 16 * WC, NW = WR * WC;
  constexpr int CI = kRealMfmaCI;  // input channels per LDS chunk
  // A chunk is CI x LR rows of the input tile (LW = TC + 2 columns with the
  // halo).  Each row is filled by one buffer load that writes LDS (lane l
  // lands at the load's LDS base + 4*l).  Rows are LC floats apart, an odd
  // multiple of 16, so the four 16-lane rows of a wave's B read fall in four
  // disjoint 16-bank groups of 64 banks (and in two of 32).  LC = 80 lets a
  // row take all 64 slots.  The RX unit has the registers for three waves
  // per SIMD but three buffers of 80-float rows leave LDS for two blocks per
  // CU: there LC = 48 and only the LW lanes of a row issue its load (the
  // rest are switched off and write nothing), which fits three.  The arrays
  // carry 64 - LC floats of tail so that a full-width row write would still
  // stay inside them.
  constexpr int LR = TR + 2, LW = TC + 2, LC = RX ? BNN_MLC_RX : BNN_MLC, LPL = LR * LC;
  constexpr bool kRowMask = LC < 64;
  constexpr int LTAIL = kRowMask ? 64 - LC : 0;
  static_assert(LW <= 64, "a tile row must fit one 64-lane load");
  static_assert(LW <= LC && LC % 16 == 0 && (LC / 16) % 2 == 1, "rows hold LW floats in odd 16-bank groups");
  constexpr int NROW = CI * LR;             // row loads per chunk
  constexpr int KR = NROW / NW;  // row loads per wave
  static_assert(NROW % NW == 0, "every wave issues the same number of row loads");
  static_assert(!RX || NW == 4, "the projection rows of a chunk are one per wave of four");
  constexpr int KL = KR + (RX ? 1 : 0);  // LDS-writing loads per wave and chunk
  // Three buffers: chunk ch is read from one while ch+1 has landed in the
  // next and ch+2 is in flight into the third.
  __shared__ float tile0[CI * LPL + LTAIL], tile1[CI * LPL + LTAIL], tile2[CI * LPL + LTAIL];  // [ci][row][col]
  constexpr int WL = RX ? 4 * 64 : 1;  // projection rows of a chunk (RX)
  __shared__ float wl0[WL], wl1[WL], wl2[WL];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = (wv / WC) * 4, wc = (wv % WC) * 16;
  int bid = blockIdx.x;
  const int tx = bid % tilesW;
  bid /= tilesW;
  const int ty = bid % tilesH;
  const int n = bid / tilesH;
  const int y0 = ty * TR, x0 = tx * TC;
  const int g = blockIdx.y;  // 16-channel group
  const int HW = a.H * a.W;
  // the lane's four output channels: 16g + 4*(lane/16) + k
  const int cq = g * 16 + 4 * (lane >> 4);

  // Row load (ci, r) of chunk ch reads input channel ch*CI + ci, image row
  // y0 - 1 + r: the lane part of its byte offset is the column, the rest is
  // scalar.  A column outside the image or past the halo gets the lane
  // offset kFar, a row outside the image (or a channel past cin in the last
  // chunk) the scalar offset kFar: with the input under kFar bytes either
  // sum lies past the buffer (both together stay below 2^32), so those
  // positions read 0.  A product w * 0 adds +-0 to a chain that never holds
  // -0, which leaves it unchanged, so every chunk runs all CI channels.
  const InGeom ig = in_geom(a, n);
  const int gx = x0 - 1 + lane;
  const uint32_t vo_lane =
      (lane < LW && gx >= 0 && gx < ig.xlim) ? (uint32_t)(ig.base + (size_t)gx) * 4u : kRealFar;
  const uint32_t cs4 = (uint32_t)__builtin_amdgcn_readfirstlane((int)(ig.cstride * 4u));
  const uint32_t rs4 = (uint32_t)__builtin_amdgcn_readfirstlane(ig.rstride * 4);
  // tile rows [rlo, rhi) lie inside the image
  const int rlo = y0 == 0 ? 1 : 0;
  const int rhi = min(LR, __builtin_amdgcn_readfirstlane(ig.ylim) - y0 + 1);
  const int nchunk = (a.cin + CI - 1) / CI;
  typedef __attribute__((address_space(3))) float* lds_f32;
  // the three chunk buffers by compile-time index (distinct variables, so
  // the compiler can tell a buffer being read from one being filled)
  auto bufp = [&](auto bc) -> float* {
    constexpr int B = decltype(bc)::value;
    if constexpr (B == 0) return tile0;
    else if constexpr (B == 1) return tile1;
    else return tile2;
  };
  auto wlp = [&](auto bc) -> float* {
    constexpr int B = decltype(bc)::value;
    if constexpr (B == 0) return wl0;
    else if constexpr (B == 1) return wl1;
    else return wl2;
  };
  // wave wv fills the KR / LR channels [wv*KR/LR, ...) of the chunk
  static_assert(KR % LR == 0, "a wave's row loads cover whole channels");
  // The LDS-writing loads are issued from inline assembly, so the compiler
  // does not track them: its own wait placement assumes any pending LDS
  // write may alias any LDS read and would wait for the chunk after next
  // before reading this one.  The waits for them are explicit (step).
  const uint64_t xaddr = (uint64_t)(uintptr_t)a.x;
  const u32x4 rsrc = {(uint32_t)xaddr, (uint32_t)(xaddr >> 32) & 0xFFFFu, xbytes, 0x00020000u};
  const uint64_t paddr = RX ? (uint64_t)(uintptr_t)a.pw : 0;
  const u32x4 psrc = {(uint32_t)paddr, (uint32_t)(paddr >> 32) & 0xFFFFu,
                      RX ? (uint32_t)(gridDim.y * nchunk * 4 * 64 * 4) : 0u, 0x00020000u};
  auto issue = [&](auto bc, int ch) {
    // the row arithmetic stays here rather than being hoisted out of the
    // chunk loop, where its 3 x KR scalars would not fit in registers
    int cw0 = wv * (KR / LR);
    asm volatile("" : "+s"(cw0));
    const uint32_t dst = (uint32_t)(uintptr_t)(lds_f32)(bufp(bc)) + (uint32_t)(cw0 * LPL * 4);
    auto rows = [&] {
#pragma unroll
      for (int j = 0; j < KR / LR; ++j) {
        const int cin_j = ch * CI + cw0 + j;  // input channel of these rows
        const bool chan_ok = !PARTIAL || cin_j < a.cin;
        const uint32_t cbase = (uint32_t)cin_j * cs4 + (uint32_t)(y0 - 1) * rs4;
#pragma unroll
        for (int r = 0; r < LR; ++r) {
          const bool ok = chan_ok && r >= rlo && r < rhi;
          const uint32_t soff = ok ? cbase + (uint32_t)r * rs4 : kRealFar;
          const uint32_t m0v =
              (uint32_t)__builtin_amdgcn_readfirstlane((int)(dst + (uint32_t)((j * LPL + r * LC) * 4)));
          const uint32_t vl = vo_lane;
          const u32x4 rd = rsrc;
          asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds"
                       :
                       : "s"(m0v), "v"(vl), "s"(rd), "s"(soff)
                       : "memory");
        }
      }
    };
    // one lane-masked region for all of the wave's row loads
    if (!kRowMask || lane < LW) rows();
    if constexpr (RX) {
      // this wave's projection row of the chunk (lane l -> slot 64*wv + l)
      const uint32_t m0v = (uint32_t)__builtin_amdgcn_readfirstlane(
          (int)((uint32_t)(uintptr_t)(lds_f32)(wlp(bc)) + (uint32_t)(wv * 256)));
      const uint32_t soff = (uint32_t)__builtin_amdgcn_readfirstlane((int)((((uint32_t)g * nchunk + ch) * 4 + wv) * 256u));
      const uint32_t vl = (uint32_t)lane * 4u;
      const u32x4 rd = psrc;
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds"
                   :
                   : "s"(m0v), "v"(vl), "s"(rd), "s"(soff)
                   : "memory");
    }
  };

  // RX: acc[0] the conv chain, acc[1] the projection chain
  constexpr int NACC = RX ? 2 : 9;
  f32x16 acc[NACC];
#pragma unroll
  for (int t = 0; t < NACC; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[t][r] = 0.0f;

  // the weight masks through the constant address space: the kernel never
  // writes them, and saying so keeps their loads scalar next to the
  // LDS-writing buffer loads
  typedef const __attribute__((address_space(4))) uint64_t* const_u64;
  const_u64 wm = (const_u64)a.wm + (size_t)g * nchunk * CI * 3;
  const int lb = (wr + (lane >> 4)) * LC + wc + (lane & 15);
  // One chunk of CI channels on the matrix cores.  The chunk's weight masks
  // arrive in one scalar batch; channel cl+1's inputs are read while channel
  // cl's nine products run (the scheduling barriers keep the compiler from
  // moving the reads next to their use).
  auto run_chunk = [&](auto bc, int ch) {
    const int ci0 = ch * CI;
    const float* tb = bufp(bc) + lb;
    uint64_t mk[CI][3];
#pragma unroll
    for (int cl = 0; cl < CI; ++cl)
#pragma unroll
      for (int q = 0; q < 3; ++q) mk[cl][q] = wm[(size_t)(ci0 + cl) * 3 + q];
    float xb[2][9];
#pragma unroll
    for (int t = 0; t < 9; ++t) xb[0][t] = tb[(t / 3) * LC + t % 3];
#pragma unroll
    for (int cl = 0; cl < CI; ++cl) {
      float wa[3];
#pragma unroll
      for (int q = 0; q < 3; ++q) wa[q] = __builtin_amdgcn_inverse_ballot_w64(mk[cl][q]) ? 1.0f : -1.0f;
      if (cl + 1 < CI) {
#pragma unroll
        for (int t = 0; t < 9; ++t) xb[(cl + 1) & 1][t] = tb[(cl + 1) * LPL + (t / 3) * LC + t % 3];
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (RX) {
        // the projection step (weights of channels 4q..4q+3 in one
        // register, block cl%4 broadcast) sits inside the conv chain, whose
        // steps wait on each other
        const float pa = wlp(bc)[(cl >> 2) * 64 + lane];
        mfma_chain(acc[0], wa, xb[cl & 1], std::make_integer_sequence<int, 4>{});
        // (the broadcast block must be a literal; the switch folds once unrolled)
        switch (cl & 3) {
          case 0: acc[1] = __builtin_amdgcn_mfma_f32_16x16x1f32(pa, xb[cl & 1][4], acc[1], 2, 0, 0); break;
          case 1: acc[1] = __builtin_amdgcn_mfma_f32_16x16x1f32(pa, xb[cl & 1][4], acc[1], 2, 1, 0); break;
          case 2: acc[1] = __builtin_amdgcn_mfma_f32_16x16x1f32(pa, xb[cl & 1][4], acc[1], 2, 2, 0); break;
          default: acc[1] = __builtin_amdgcn_mfma_f32_16x16x1f32(pa, xb[cl & 1][4], acc[1], 2, 3, 0); break;
        }
        mfma_chain_tap<4>(acc[0], wa, xb[cl & 1]);
        mfma_chain_tap<5>(acc[0], wa, xb[cl & 1]);
        mfma_chain_tap<6>(acc[0], wa, xb[cl & 1]);
        mfma_chain_tap<7>(acc[0], wa, xb[cl & 1]);
        mfma_chain_tap<8>(acc[0], wa, xb[cl & 1]);
      } else {
        mfma_taps(acc, wa, xb[cl & 1], std::make_integer_sequence<int, 9>{});
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // The chunk barrier: this wave's own waits (below) make its LDS-writing
  // loads complete, and every LDS read of the chunk has fed an MFMA before
  // the barrier, so no memory fence is needed (a fence would wait for the
  // loads still in flight for the chunk after next); the signal fences keep
  // the compiler from moving LDS accesses across it.
  auto chunk_barrier = [] {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  };
  // s_waitcnt with vmcnt <= KL or 0 (expcnt and lgkmcnt left alone)
  constexpr int kWaitKD = (KL & 15) | ((KL >> 4) << 14) | (7 << 4) | (15 << 8);
  constexpr int kWait0 = (7 << 4) | (15 << 8);
  static_assert(KL < 64, "vmcnt holds at most 63");
  // Chunk ch from buffer B; chunk ch+2, if any, is fetched into buffer
  // B+2 (mod 3), last read as chunk ch-1, which every wave finished before
  // the last barrier.  Then this wave's loads of chunk ch+1, issued one step
  // earlier, are waited for (only the KL loads of chunk ch+2 may remain) and
  // the barrier makes every wave's loads visible.
  auto step = [&](auto bc, int ch) {
    constexpr int B = decltype(bc)::value;
    const bool ahead = ch + 2 < nchunk;
    if (ahead) issue(std::integral_constant<int, (B + 2) % 3>{}, ch + 2);
    run_chunk(bc, ch);
    if (ahead) __builtin_amdgcn_s_waitcnt(kWaitKD);
    else __builtin_amdgcn_s_waitcnt(kWait0);
    chunk_barrier();
  };
  issue(std::integral_constant<int, 0>{}, 0);
  if (nchunk > 1) {
    issue(std::integral_constant<int, 1>{}, 1);
    __builtin_amdgcn_s_waitcnt(kWaitKD);
  } else {
    __builtin_amdgcn_s_waitcnt(kWait0);
  }
  chunk_barrier();
  // chunk c lives in buffer c % 3
  int ch = 0;
#pragma unroll 1
  for (; ch + 3 <= nchunk; ch += 3) {
    step(std::integral_constant<int, 0>{}, ch);
    step(std::integral_constant<int, 1>{}, ch + 1);
    step(std::integral_constant<int, 2>{}, ch + 2);
  }
  if (ch < nchunk) {
    step(std::integral_constant<int, 0>{}, ch);
    if (ch + 1 < nchunk) step(std::integral_constant<int, 1>{}, ch + 1);
  }

  // alpha and fold parameters of the lane's four channels (the arrays are
  // padded to 32 channels)
  float p_al[4], p_A[4], p_B[4], p_sl[4], p_rs[4];
  if constexpr (RX) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      p_al[k] = a.alpha[cq + k];
      p_A[k] = a.A[cq + k];
      p_B[k] = a.B[cq + k];
      p_sl[k] = a.slope[cq + k];
      p_rs[k] = a.rsign[cq + k];
    }
    const int xo = x0 + wc + (lane & 15);
    const size_t plane = (size_t)(a.ntot ? a.ntot : a.N) * HW;
    uint32_t w01 = 0, w23 = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int k = r & 3, b = r >> 2;
      const int y = y0 + wr + b;
      const int co = cq + k;
      const bool in = y < a.H && xo < a.W && co < a.cout;
      const float c = __fmul_rn(p_al[k], acc[0][r]);
      const float res = acc[1][r];
      const size_t at = ((size_t)n * a.cout + co) * HW + (size_t)y * a.W + xo;
      if (a.f32 && in) a.f32[at] = c;
      if (a.f32b && in) a.f32b[at] = res;
      const float t = __fadd_rn(__fmaf_rn(p_A[k], c, p_B[k]), res);
      const float h = t >= 0.0f ? t : __fmul_rn(p_sl[k], t);
      if (in) a.hout[(size_t)co * plane + ((size_t)n * a.H + y) * a.W + xo] = h;
      const uint32_t bit = (__fadd_rn(h, p_rs[k]) > 0.0f && co < a.cout) ? 1u : 0u;
      const int sh = 16 * (b & 1) + 4 * (lane >> 4) + k;
      if (b < 2) w01 |= bit << sh;
      else w23 |= bit << sh;
    }
    if (!a.out) return;
    w01 |= (uint32_t)__shfl_xor((int)w01, 16);
    w01 |= (uint32_t)__shfl_xor((int)w01, 32);
    w23 |= (uint32_t)__shfl_xor((int)w23, 16);
    w23 |= (uint32_t)__shfl_xor((int)w23, 32);
    const int q = lane >> 4;
    const uint32_t word = ((q < 2 ? w01 : w23) >> (16 * (q & 1))) & 0xFFFFu;
    const int y = y0 + wr + q;
    if (y >= a.H || xo >= a.W) return;
    const int cwo = (a.cout + 31) >> 5;
    uint8_t* dst = reinterpret_cast<uint8_t*>(a.out + ((size_t)n * HW + (size_t)y * a.W + xo) * cwo) + g * 2;
    if ((g & 1) == 0 && g == (int)gridDim.y - 1) *reinterpret_cast<uint32_t*>(dst) = word;
    else *reinterpret_cast<uint16_t*>(dst) = (uint16_t)word;
    return;
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    p_al[k] = a.alpha[cq + k];
    if (a.out) {
      p_A[k] = a.A[cq + k];
      p_B[k] = a.B[cq + k];
      p_sl[k] = a.slope[cq + k];
      p_rs[k] = a.rsign[cq + k];
    }
  }

  // taps in row-major order into acc (an out-of-image tap summed zeros to
  // +0 and leaves it unchanged), alpha, then the real fold
  // (csrc/bnn_fold.c:62-77): z = fma(A, x, B); z<0 -> slope*z; r = z + rsign;
  // bit = r > 0.  The reference build fuses A*x+B only.  Register r of lane
  // l is pixel row r/4, channel 4*(l/16) + r%4: each lane builds the nibble
  // of its four channels for each of its four pixels, and two xor shuffles
  // gather the 16-bit words of all four pixels in every lane of a column.
  const int xo = x0 + wc + (lane & 15);
  uint32_t w01 = 0, w23 = 0;  // pixel rows 0,1 / 2,3: 16 bits each
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    float v = 0.0f;
#pragma unroll
    for (int t = 0; t < 9; ++t) v = __fadd_rn(v, acc[t][r]);
    const int k = r & 3, b = r >> 2;
    const int y = y0 + wr + b;
    const int co = cq + k;
    const float o = __fmul_rn(p_al[k], v);
    if (a.f32 && y < a.H && xo < a.W && co < a.cout)
      a.f32[((size_t)n * a.cout + co) * HW + (size_t)y * a.W + xo] = o;
    if (a.out) {
      float z = __fmaf_rn(p_A[k], o, p_B[k]);
      if (z < 0.0f) z = __fmul_rn(p_sl[k], z);
      const float rr = __fadd_rn(z, p_rs[k]);
      const uint32_t bit = (rr > 0.0f && co < a.cout) ? 1u : 0u;
      const int sh = 16 * (b & 1) + 4 * (lane >> 4) + k;
      if (b < 2) w01 |= bit << sh;
      else w23 |= bit << sh;
    }
  }
  if (!a.out) return;
  w01 |= (uint32_t)__shfl_xor((int)w01, 16);
  w01 |= (uint32_t)__shfl_xor((int)w01, 32);
  w23 |= (uint32_t)__shfl_xor((int)w23, 16);
  w23 |= (uint32_t)__shfl_xor((int)w23, 32);
  // lane group q stores pixel row q of its column.  Group g owns bits
  // [16g, 16g+16) of the pixel: a 16-bit store, or the whole word (upper
  // half 0) when it is the last group and starts a word.
  const int q = lane >> 4;
  const uint32_t word = ((q < 2 ? w01 : w23) >> (16 * (q & 1))) & 0xFFFFu;
  const int y = y0 + wr + q;
  if (y >= a.H || xo >= a.W) return;
  const int cwo = (a.cout + 31) >> 5;
  uint8_t* dst = reinterpret_cast<uint8_t*>(a.out + ((size_t)n * HW + (size_t)y * a.W + xo) * cwo) + g * 2;
  if ((g & 1) == 0 && g == (int)gridDim.y - 1) *reinterpret_cast<uint32_t*>(dst) = word;
  else *reinterpret_cast<uint16_t*>(dst) = (uint16_t)word;
}

// ------------------------------------------------------------------------
// real-input conv on the matrix cores, persistent, 16-byte staging
// ------------------------------------------------------------------------
// The same per-tap K = 1 MFMA chains, weight masks and epilogue as
// k_real_mfma<2, 2> (8 x 32 output tile per block, 4 waves of 4 x 16
// pixels, 16 channels per group), for inputs whose row width is a multiple
// of 4, with two changes to the input staging:
//  * Each lane's LDS-writing load moves 16 bytes (4 columns), so a chunk of
//    8 channels x 10 tile rows is 15 loads per block instead of 80.  A tile
//    row is 10 such slots, image columns x0-4 .. x0+35 (the 34 the taps
//    read sit at 3..36), padded to 12 slots = 48 floats, 16 mod 32: the
//    four 16-lane rows of an operand read fall in disjoint bank groups of
//    each half-wave.  A slot outside the image, or a pad slot, takes the
//    offset kFar and lands as zeros.  The load's LDS address is
//    M0 + 16 * lane, so slot s of a chunk (row s / 12, slot s % 12) is byte
//    16 s of its buffer and the 960 slots are 15 contiguous 1 KiB loads,
//    load k issued by wave k % 4.
//  * Persistent blocks walk tiles blockIdx.x, +gridDim.x, ...; the chunk
//    pipeline (three buffers: one read, one landed, one in flight) runs
//    across tile boundaries, so a tile's first chunks arrive during the
//    previous tile's last ones and its epilogue.
// Measured against reading the weights as per-lane floats from LDS (three
// more LDS reads per channel instead of three selects): the selects are
// faster.  Every helper lambda is forced inline: one left out of line takes
// the accumulators by reference, which puts them in scratch memory for the
// whole kernel.
#ifndef BNN_R4ROWF
#define BNN_R4ROWF 48
#endif
constexpr int kR4RowF = BNN_R4ROWF;                  // floats per LDS tile row
constexpr int kR4Slots = kR4RowF / 4;                // 16-byte slots per row
constexpr int kR4Rows = kRealMfmaCI * 10;            // tile rows per chunk
constexpr int kR4Ld = kR4Rows * kR4Slots / 64;       // loads per chunk
constexpr int kR4LdW = (kR4Ld + 3) / 4;              // loads per wave (at most)
constexpr int kR4BufF = kR4Ld * 256;                 // floats per buffer
static_assert(kR4Rows * kR4Slots % 64 == 0, "whole 1 KiB loads per chunk");
static_assert(kR4RowF % 32 == 16 && kR4Slots >= 10, "rows of 10 slots, 16 mod 32 floats apart");

template <bool PARTIAL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void k_real_mfma4(const RealArgs a, uint32_t xbytes, int tilesH, int tilesW, int ntile) {
  constexpr int CI = kRealMfmaCI, LR = 10, TR = 8, TC = 32, LPL = LR * kR4RowF;
  __shared__ __attribute__((aligned(16))) float buf[3 * kR4BufF];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = (wv >> 1) * 4, wc = (wv & 1) * 16;
  const int g = blockIdx.y;
  const int nchunk = (a.cin + CI - 1) / CI;
  const int t0 = blockIdx.x, tstep = gridDim.x;
  const int mytiles = t0 < ntile ? (ntile - t0 + tstep - 1) / tstep : 0;
  const int total = mytiles * nchunk;
  if (total == 0) return;
  const int cq = g * 16 + 4 * (lane >> 4);
  // this wave's loads k = wv + 4m < 15
  const int nld = (kR4Ld - wv + 3) / 4;
  // per row load m: the lane's slot -> channel lcl, tile row lr and column
  // group lj; rel is the slot's element offset from the tile's first row and
  // column group.  A pad slot, or a slot past the chunk's loads, gets a row
  // far outside every image, so the per-tile test below rejects it.  (Plain
  // integers: per-lane flags would each take a scalar register pair.)
  const InGeom ig0 = in_geom(a, 0);
  const uint32_t cstr = (uint32_t)ig0.cstride, rstr = (uint32_t)ig0.rstride;
  int lcl[kR4LdW], lr[kR4LdW], lj4[kR4LdW];
  uint32_t rel[kR4LdW];
#pragma unroll
  for (int m = 0; m < kR4LdW; ++m) {
    const int k = wv + 4 * m;
    const int sl = k * 64 + lane, row = sl / kR4Slots, j = sl - row * kR4Slots;
    lcl[m] = row / LR;
    lr[m] = (k < kR4Ld && j < 10) ? row - lcl[m] * LR : -(1 << 20);
    lj4[m] = 4 * j;
    rel[m] = (uint32_t)lcl[m] * cstr + (uint32_t)(row - lcl[m] * LR) * rstr + (uint32_t)(4 * j);
  }
  const uint32_t cs4 = (uint32_t)__builtin_amdgcn_readfirstlane((int)(cstr * 4u));
  // lane part of the byte offset of each row load for tile t (kRealFar
  // where the slot lies outside the image or is a pad slot); the sums wrap
  // modulo 2^32 and are exact for the slots inside the image
  auto tile_offsets = [&](int t, uint32_t (&lo)[kR4LdW]) __attribute__((always_inline)) {
    const int tx = t % tilesW, rest = t / tilesW, ty = rest % tilesH, n = rest / tilesH;
    const InGeom ig = in_geom(a, n);
    const int y0 = ty * TR, x0 = tx * TC;
    const uint32_t org = (uint32_t)ig.base + (uint32_t)(y0 - 1) * rstr + (uint32_t)(x0 - 4);
#pragma unroll
    for (int m = 0; m < kR4LdW; ++m) {
      const uint32_t iy = (uint32_t)(y0 - 1 + lr[m]), ix = (uint32_t)(x0 - 4 + lj4[m]);
      const bool ok = (iy < (uint32_t)ig.ylim) & (ix < (uint32_t)ig.xlim);
      lo[m] = ok ? (org + rel[m]) * 4u : kRealFar;
    }
  };
  const uint64_t xaddr = (uint64_t)(uintptr_t)a.x;
  // (every word through readfirstlane: the descriptors must live in SGPRs)
  auto uni = [](uint32_t v) __attribute__((always_inline)) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); };
  const u32x4 xsrc = {uni((uint32_t)xaddr), uni((uint32_t)(xaddr >> 32) & 0xFFFFu), uni(xbytes), 0x00020000u};
  typedef __attribute__((address_space(3))) float* lds_f32;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_f32)buf;
  // chunk ch of the tile whose row offsets are lo, into buffer B
  auto issue = [&](int b, int ch, const uint32_t (&lo)[kR4LdW]) __attribute__((always_inline)) {
    const uint32_t dst = lds0 + (uint32_t)(b * kR4BufF * 4);
    const uint32_t sx = (uint32_t)__builtin_amdgcn_readfirstlane((int)((uint32_t)(ch * CI) * cs4));
#pragma unroll
    for (int m = 0; m < kR4LdW; ++m) {
      const int k = wv + 4 * m;
      if (k >= kR4Ld) break;
      const uint32_t m0v = (uint32_t)__builtin_amdgcn_readfirstlane((int)(dst + (uint32_t)(k * 1024)));
      uint32_t vo = lo[m];
      if (PARTIAL && lcl[m] >= a.cin - ch * CI) vo = kRealFar;
      const u32x4 rd = xsrc;
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                   :
                   : "s"(m0v), "v"(vo), "s"(rd), "s"(sx)
                   : "memory");
    }
  };

  f32x16 acc[9];
#pragma unroll
  for (int t = 0; t < 9; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[t][r] = 0.0f;
  // the lane's operand base in a buffer: tile row wr + lane/16, LDS column
  // wc + lane%16 + 3 (image column x0 + wc + lane%16 - 1)
  const int lb = (wr + (lane >> 4)) * kR4RowF + wc + (lane & 15) + 3;
  // the weight masks through the constant address space (scalar loads)
  typedef const __attribute__((address_space(4))) uint64_t* const_u64;
  const const_u64 wm = (const_u64)a.wm + (size_t)g * nchunk * CI * 3;
  auto run_chunk = [&](auto bc, int ch) __attribute__((always_inline)) {
    const float* tb = buf + decltype(bc)::value * kR4BufF + lb;
    uint64_t mk[CI][3];
#pragma unroll
    for (int cl = 0; cl < CI; ++cl)
#pragma unroll
      for (int q = 0; q < 3; ++q) mk[cl][q] = wm[(size_t)(ch * CI + cl) * 3 + q];
    float xb[2][9];
#pragma unroll
    for (int t = 0; t < 9; ++t) xb[0][t] = tb[(t / 3) * kR4RowF + t % 3];
#pragma unroll
    for (int cl = 0; cl < CI; ++cl) {
      float wa[3];
#pragma unroll
      for (int q = 0; q < 3; ++q) wa[q] = __builtin_amdgcn_inverse_ballot_w64(mk[cl][q]) ? 1.0f : -1.0f;
      if (cl + 1 < CI) {
#pragma unroll
        for (int t = 0; t < 9; ++t) xb[(cl + 1) & 1][t] = tb[(cl + 1) * LPL + (t / 3) * kR4RowF + t % 3];
      }
      __builtin_amdgcn_sched_barrier(0);
      mfma_taps(acc, wa, xb[cl & 1], std::make_integer_sequence<int, 9>{});
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto chunk_barrier = []() __attribute__((always_inline)) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  };
  // wait until only this wave's loads of the newest chunk may be in flight
  constexpr int kWaitHi = (kR4LdW & 15) | (7 << 4) | (15 << 8), kWaitLo = ((kR4LdW - 1) & 15) | (7 << 4) | (15 << 8);
  static_assert(kR4LdW < 16, "vmcnt field");
  auto wait_landed = [&](bool newest_in_flight) __attribute__((always_inline)) {
    if (!newest_in_flight) __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
    else if (nld == kR4LdW) __builtin_amdgcn_s_waitcnt(kWaitHi);
    else __builtin_amdgcn_s_waitcnt(kWaitLo);
  };

  // alpha and fold parameters of the lane's four channels, the same for
  // every tile (arrays padded to 32 channels)
  float p_al[4], p_A[4], p_B[4], p_sl[4], p_rs[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    p_al[k] = a.alpha[cq + k];
    if (a.out) {
      p_A[k] = a.A[cq + k];
      p_B[k] = a.B[cq + k];
      p_sl[k] = a.slope[cq + k];
      p_rs[k] = a.rsign[cq + k];
    }
  }
  const int HW = a.H * a.W;
  // the tile's taps summed in row-major order, alpha, the real fold, bits
  // (the k_real_mfma epilogue; csrc/bnn_conv_realin.c:99-111,
  // csrc/bnn_fold.c:62-77)
  auto epilogue = [&](int t) __attribute__((always_inline)) {
    const int tx = t % tilesW, rest = t / tilesW, ty = rest % tilesH, n = rest / tilesH;
    const int y0 = ty * TR, x0 = tx * TC;
    const int xo = x0 + wc + (lane & 15);
    uint32_t w01 = 0, w23 = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float v = 0.0f;
#pragma unroll
      for (int tp = 0; tp < 9; ++tp) v = __fadd_rn(v, acc[tp][r]);
      const int k = r & 3, b = r >> 2;
      const int y = y0 + wr + b;
      const int co = cq + k;
      const float o = __fmul_rn(p_al[k], v);
      if (a.f32 && y < a.H && xo < a.W && co < a.cout)
        a.f32[((size_t)n * a.cout + co) * HW + (size_t)y * a.W + xo] = o;
      if (a.out) {
        float z = __fmaf_rn(p_A[k], o, p_B[k]);
        if (z < 0.0f) z = __fmul_rn(p_sl[k], z);
        const float rr = __fadd_rn(z, p_rs[k]);
        const uint32_t bit = (rr > 0.0f && co < a.cout) ? 1u : 0u;
        const int sh = 16 * (b & 1) + 4 * (lane >> 4) + k;
        if (b < 2) w01 |= bit << sh;
        else w23 |= bit << sh;
      }
    }
    if (!a.out) return;
    w01 |= (uint32_t)__shfl_xor((int)w01, 16);
    w01 |= (uint32_t)__shfl_xor((int)w01, 32);
    w23 |= (uint32_t)__shfl_xor((int)w23, 16);
    w23 |= (uint32_t)__shfl_xor((int)w23, 32);
    const int q = lane >> 4;
    const uint32_t word = ((q < 2 ? w01 : w23) >> (16 * (q & 1))) & 0xFFFFu;
    const int y = y0 + wr + q;
    if (y >= a.H || xo >= a.W) return;
    const int cwo = (a.cout + 31) >> 5;
    uint8_t* dst = reinterpret_cast<uint8_t*>(a.out + ((size_t)n * HW + (size_t)y * a.W + xo) * cwo) + g * 2;
    if ((g & 1) == 0 && g == (int)gridDim.y - 1) *reinterpret_cast<uint32_t*>(dst) = word;
    else *reinterpret_cast<uint16_t*>(dst) = (uint16_t)word;
  };

  // The issue position runs two chunks ahead of the compute position, so
  // the last two steps of a tile issue the next tile's first two chunks.
  // Row offsets of the current and the next tile are computed once per tile,
  // outside the chunk loop (kept out of it, the address arithmetic takes
  // the scalar registers the loop needs).  Chunk c of a tile lives in
  // buffer c % 3: with nchunk a multiple of 3 every tile starts in buffer 0
  // and each read's buffer is a compile-time constant.
  uint32_t lo_cur[kR4LdW], lo_nxt[kR4LdW];
  tile_offsets(t0, lo_cur);
  if (mytiles > 1) tile_offsets(t0 + tstep, lo_nxt);
  issue(0, 0, lo_cur);
  if (nchunk > 1) issue(1, 1, lo_cur);
  else if (mytiles > 1) issue(1, 0, lo_nxt);
  wait_landed(total > 1);
  chunk_barrier();
  int gc = 0;
  auto step = [&](auto bc, int ch) __attribute__((always_inline)) {
    constexpr int B = decltype(bc)::value;
    const bool ahead = gc + 2 < total;
    if (ahead) {
      if (ch + 2 < nchunk) issue((B + 2) % 3, ch + 2, lo_cur);
      else issue((B + 2) % 3, ch + 2 - nchunk, lo_nxt);
    }
    run_chunk(bc, ch);
    wait_landed(ahead);
    chunk_barrier();
    ++gc;
  };
#pragma unroll 1
  for (int tc = 0; tc < mytiles; ++tc) {
#pragma unroll 1
    for (int ch = 0; ch < nchunk; ch += 3) {
      step(std::integral_constant<int, 0>{}, ch);
      step(std::integral_constant<int, 1>{}, ch + 1);
      step(std::integral_constant<int, 2>{}, ch + 2);
    }
    epilogue(t0 + tc * tstep);
#pragma unroll
    for (int tp = 0; tp < 9; ++tp)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[tp][r] = 0.0f;
#pragma unroll
    for (int m = 0; m < kR4LdW; ++m) lo_cur[m] = lo_nxt[m];
    if (tc + 2 < mytiles) tile_offsets(t0 + (tc + 2) * tstep, lo_nxt);
  }
}

// 1x1 real-input stem on the matrix cores (v2 models)
// ------------------------------------------------------------------------
// out[co][p] = alpha[co] * (sum over ci from 0 in order of w[co][ci] * x[ci][p])
// (csrc/bnn_conv_realin.c:140-155), then the real fold, as bits.  One
// v_mfma_f32_16x16x1_4b_f32 per (ci, 16-channel group, pixel set) advances
// 16 channels x 64 pixels by one exact fma step (w is +1, -1 or 0, so w*x is
// exact and fma(w, x, acc) rounds as acc + w*x does).  A wave owns 64*PX
// consecutive pixels: lane l loads pixels PX*l .. PX*l+PX-1 of each input
// channel with one PX-dword load (the wave reads 256*PX contiguous bytes),
// and MFMA pass p takes component p, so its B block b, column j is pixel
// PX*(16b+j)+p.  With CBSZ = 2 one weight register holds the signs of four
// input channels (lanes 16k..16k+15 = channel 4q+k), built from two lane
// masks (positive, nonzero).  D register r of lane l in pass p holds pixel
// PX*(16*(r/4) + l%16) + p, channel 16g + 4*(l/16) + r%4.

template <int PX>
struct StemVec;
template <>
struct StemVec<1> {
  float v[1];
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
    v[0] = ld_f32(rs, voff, soff);
  }
};
template <>
struct StemVec<2> {
  float v[2];
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
    const stem_f32x2 r = raw_load_f32x2(rs, (int)voff, (int)soff, 0);
    v[0] = r[0];
    v[1] = r[1];
  }
};
template <>
struct StemVec<4> {
  float v[4];
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
    const stem_f32x4 r = raw_load_f32x4(rs, (int)voff, (int)soff, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = r[i];
  }
};

// f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>)
template <class F, int... H>
__device__ __forceinline__ void static_for(F&& f, std::integer_sequence<int, H...>) {
  (f(std::integral_constant<int, H>{}), ...);
}

template <int G, int PX, int T>
__device__ __forceinline__ void stem_step(f32x16 (&acc)[G][PX], const float (&wq)[G], const StemVec<PX>& xv) {
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int p = 0; p < PX; ++p)
      acc[g][p] = __builtin_amdgcn_mfma_f32_16x16x1f32(wq[g], xv.v[p], acc[g][p], 2, T, 0);
}

struct alignas(16) StemMask {
  uint64_t pos, nz;
};

// weights of quad q: masks [nq][ngp] (real_stem_masks), this wave's G groups
template <int G>
__device__ __forceinline__ void stem_weights(const uint64_t* __restrict__ wm, int q, int ngp, int g0,
                                             float (&wq)[G]) {
  const StemMask* m = reinterpret_cast<const StemMask*>(wm) + (size_t)q * ngp + g0;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const StemMask mm = m[g];
    const float sg = __builtin_amdgcn_inverse_ballot_w64(mm.pos) ? 1.0f : -1.0f;
    wq[g] = __builtin_amdgcn_inverse_ballot_w64(mm.nz) ? sg : 0.0f;
  }
}

// G channel groups per wave, PX pixels per lane, NQ quads of input channels
// in flight per lane, registers sized for OCC waves per SIMD; DUMP also
// stores the conv output as floats (a.f32).  The host guarantees that a
// lane's PX pixels lie in one row of one patch and inside or outside the
// input together.
template <int G, int PX, int NQ, int OCC, bool DUMP>
__global__ __launch_bounds__(256, OCC) void k_stem_mfma(const RealArgs a, uint32_t xbytes, int ngp) {
  const int lane = threadIdx.x & 63;
  const int ny = ngp / G;  // channel-group blocks per pixel tile
  const long tile = (long)(blockIdx.x / ny) * 4 + (threadIdx.x >> 6);
  const int g0 = (int)(blockIdx.x % ny) * G;
  const int HW = a.H * a.W;
  const long npix = (long)a.N * HW;
  const long t0 = tile * 64 * PX;   // first pixel of the wave
  const long q = t0 + PX * lane;    // this lane's first pixel in [N][H*W]
  const bool live = q < npix;
  const int n = live ? (int)(q / HW) : 0;
  const int pp = live ? (int)(q - (long)n * HW) : 0;
  const int py = pp / a.W, px = pp - py * a.W;
  const InGeom ig = in_geom(a, n);
  const bool inside = live && py < ig.ylim && px < ig.xlim;
  const uint32_t voff = inside ? (uint32_t)(ig.base + (size_t)py * ig.rstride + px) * 4u : 0x80000000u;
  const uint32_t cbytes = (uint32_t)(ig.cstride * 4u);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.x, xbytes);

  f32x16 acc[G][PX];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int p = 0; p < PX; ++p)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[g][p][r] = 0.0f;

  // Channel c sits in slot c % (4*NQ) of xr; a slot is refilled (4*NQ
  // channels ahead) right after its step has read it.  Loads run unguarded:
  // a channel at or past cin is the next image's data or past the buffer
  // (read as 0), and only the guarded tail quad can meet it.
  constexpr int kAhead = 4 * NQ;
  StemVec<PX> xr[kAhead];
#pragma unroll
  for (int k = 0; k < kAhead; ++k) xr[k].load(rs, voff, (uint32_t)k * cbytes);
  const int qf = a.cin >> 2, rem = a.cin & 3;
  auto quad = [&](auto hc, int qq) {
    constexpr int h = decltype(hc)::value;
    float wq[G];
    stem_weights<G>(a.wm, qq, ngp, g0, wq);
    stem_step<G, PX, 0>(acc, wq, xr[4 * h + 0]);
    stem_step<G, PX, 1>(acc, wq, xr[4 * h + 1]);
    stem_step<G, PX, 2>(acc, wq, xr[4 * h + 2]);
    stem_step<G, PX, 3>(acc, wq, xr[4 * h + 3]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < 4; ++k) xr[4 * h + k].load(rs, voff, (uint32_t)(4 * qq + k + kAhead) * cbytes);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto tail = [&](auto hc, int qq) {
    constexpr int h = decltype(hc)::value;
    float wq[G];
    stem_weights<G>(a.wm, qq, ngp, g0, wq);
    stem_step<G, PX, 0>(acc, wq, xr[4 * h]);
    if (rem > 1) stem_step<G, PX, 1>(acc, wq, xr[4 * h + 1]);
    if (rem > 2) stem_step<G, PX, 2>(acc, wq, xr[4 * h + 2]);
  };
  int qi = 0;
#pragma unroll 1
  for (; qi + NQ <= qf; qi += NQ)
    static_for([&](auto hc) { quad(hc, qi + decltype(hc)::value); }, std::make_integer_sequence<int, NQ>{});
  // the last qf % NQ full quads, then the partial quad (cin % 4 channels)
  static_for(
      [&](auto hc) {
        constexpr int h = decltype(hc)::value;
        if (qi + h < qf) quad(hc, qi + h);
        else if (qi + h == qf && rem) tail(hc, qi + h);
      },
      std::make_integer_sequence<int, NQ>{});

  // alpha, the real fold (csrc/bnn_fold.c:62-77, A*x+B fused as in the
  // reference build), bits gathered across the four lane groups
  const int cwo = (a.cout + 31) >> 5;
  const int ngrp = (a.cout + 15) >> 4;
  constexpr int NW = 2 * PX;  // 32-bit words of bits per lane and group
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int gg = g0 + g;
    if (gg >= ngrp) break;
    const int cq = gg * 16 + 4 * (lane >> 4);
    // pixel (b, p) = PX*(16b + l%16) + p: 16 bits at 16*((b*PX+p) % 2) of word (b*PX+p) / 2
    uint32_t wb[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) wb[i] = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int co = cq + k;
      const int cc = min(co, a.cout - 1);
      const float al = a.alpha[cc];
      const float fA = a.A[cc], fB = a.B[cc], fs = a.slope[cc], fr = a.rsign[cc];
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int p = 0; p < PX; ++p) {
          const float o = __fmul_rn(al, acc[g][p][4 * b + k]);
          const long qp = t0 + PX * (16 * b + (lane & 15)) + p;
          if (DUMP && qp < npix && co < a.cout) {
            const long nn = qp / HW;
            a.f32[((size_t)nn * a.cout + co) * HW + (qp - nn * HW)] = o;
          }
          float z = __fmaf_rn(fA, o, fB);
          if (z < 0.0f) z = __fmul_rn(fs, z);
          const float rr = __fadd_rn(z, fr);
          const uint32_t bit = (rr > 0.0f && co < a.cout) ? 1u : 0u;
          const int i = b * PX + p;
          wb[i / 2] |= bit << (16 * (i % 2) + 4 * (lane >> 4) + k);
        }
    }
    if (!a.out) continue;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      wb[i] |= (uint32_t)__shfl_xor((int)wb[i], 16);
      wb[i] |= (uint32_t)__shfl_xor((int)wb[i], 32);
    }
    // lane group b stores pixels PX*(16b + l%16) + p: 16 bits at bit
    // 16*(gg%2) of word gg/2; the last group of an odd count writes its whole word
    const int b = lane >> 4;
#pragma unroll
    for (int p = 0; p < PX; ++p) {
      uint32_t word = 0;
#pragma unroll
      for (int bb = 0; bb < 4; ++bb) {
        const int i = bb * PX + p;
        if (b == bb) word = (wb[i / 2] >> (16 * (i % 2))) & 0xFFFFu;
      }
      const long qp = t0 + PX * (16 * b + (lane & 15)) + p;
      if (qp >= npix) continue;
      uint8_t* dst = reinterpret_cast<uint8_t*>(a.out + (size_t)qp * cwo) + gg * 2;
      if ((gg & 1) == 0 && gg == ngrp - 1) *reinterpret_cast<uint32_t*>(dst) = word;
      else *reinterpret_cast<uint16_t*>(dst) = (uint16_t)word;
    }
  }
}

// ------------------------------------------------------------------------
// binary conv with fused epilogues
// ------------------------------------------------------------------------
// acc + popcount(x) as one v_bcnt_u32_b32.  Written as a chain on purpose:
// left to itself the compiler turns the per-tap sum into popcount-into-zero
// plus v_add3 trees, a quarter more VALU work for the same count.
__device__ __forceinline__ uint32_t bcnt_acc(uint32_t x, uint32_t acc) {
  uint32_t r;
  asm("v_bcnt_u32_b32 %0, %1, %2" : "=v"(r) : "v"(x), "v"(acc));
  return r;
}

template <int MT, int COG>
struct Acc {
  uint32_t d[MT * MT][COG];
};

// D[p][j] += sum over taps popcount((a ^ w) & m) for one 32-channel word.
// The weights of JB channels (9 words each, wave-uniform) are fetched as
// one batch of scalar loads before their products: fetched channel by
// channel, each would wait for its own load.
#ifndef BNN_BJB
#define BNN_BJB 8
#endif
template <int MT, int COG>
__device__ __forceinline__ void accumulate(Acc<MT, COG>& D, const uint32_t (&av)[MT + 2][MT + 2],
                                           const uint32_t (&m)[MT + 2][MT + 2],
                                           const uint32_t* __restrict__ wrow) {
  constexpr int JB = COG < BNN_BJB ? COG : BNN_BJB;
  typedef const __attribute__((address_space(4))) uint32_t* const_u32;
  const const_u32 wr = (const_u32)wrow;
#pragma unroll
  for (int j0 = 0; j0 < COG; j0 += JB) {
    uint32_t w9[JB][9];
#pragma unroll
    for (int jj = 0; jj < JB; ++jj)
#pragma unroll
      for (int t = 0; t < 9; ++t) w9[jj][t] = wr[(j0 + jj) * 9 + t];
#pragma unroll
    for (int jj = 0; jj < JB; ++jj) {
      const int j = j0 + jj;
#pragma unroll
      for (int py = 0; py < MT; ++py)
#pragma unroll
        for (int px = 0; px < MT; ++px) {
          uint32_t d = D.d[py * MT + px][j];
#pragma unroll
          for (int ky = 0; ky < 3; ++ky)
#pragma unroll
            for (int kx = 0; kx < 3; ++kx)
              d = bcnt_acc((av[py + ky][px + kx] ^ w9[jj][ky * 3 + kx]) & m[py + ky][px + kx], d);
          D.d[py * MT + px][j] = d;
        }
    }
  }
}

// The same for an input of at most 16 channels (one word per pixel, the
// high half zero): the words (and masks) of taps 2p and 2p+1 are packed into
// one, tap 8 alone, and the weights come packed the same way (5 words per
// channel), so each output channel takes 5 popcounts instead of 9.
template <int MT, int COG>
__device__ __forceinline__ void accumulate_pair(Acc<MT, COG>& D, const uint32_t (&av)[MT + 2][MT + 2],
                                                const uint32_t (&m)[MT + 2][MT + 2],
                                                const uint32_t* __restrict__ wrow) {
  constexpr int JB = COG < BNN_BJB ? COG : BNN_BJB;
  typedef const __attribute__((address_space(4))) uint32_t* const_u32;
  const const_u32 wr = (const_u32)wrow;
  uint32_t c[MT * MT][5], mm[MT * MT][5];
#pragma unroll
  for (int py = 0; py < MT; ++py)
#pragma unroll
    for (int px = 0; px < MT; ++px)
#pragma unroll
      for (int q = 0; q < 5; ++q) {
        const int t0 = 2 * q, t1 = 2 * q + 1;
        const uint32_t a0 = av[py + t0 / 3][px + t0 % 3], m0 = m[py + t0 / 3][px + t0 % 3];
        if (t1 < 9) {
          const uint32_t a1 = av[py + t1 / 3][px + t1 % 3], m1 = m[py + t1 / 3][px + t1 % 3];
          c[py * MT + px][q] = a0 | (a1 << 16);
          mm[py * MT + px][q] = (m0 & 0xFFFFu) | (m1 & 0xFFFF0000u);
        } else {
          c[py * MT + px][q] = a0;
          mm[py * MT + px][q] = m0;
        }
      }
#pragma unroll
  for (int j0 = 0; j0 < COG; j0 += JB) {
    uint32_t w5[JB][5];
#pragma unroll
    for (int jj = 0; jj < JB; ++jj)
#pragma unroll
      for (int q = 0; q < 5; ++q) w5[jj][q] = wr[(j0 + jj) * 5 + q];
#pragma unroll
    for (int jj = 0; jj < JB; ++jj)
#pragma unroll
      for (int p = 0; p < MT * MT; ++p) {
        uint32_t d = D.d[p][j0 + jj];
#pragma unroll
        for (int q = 0; q < 5; ++q) d = bcnt_acc((c[p][q] ^ w5[jj][q]) & mm[p][q], d);
        D.d[p][j0 + jj] = d;
      }
  }
}

template <int NP>
__device__ __forceinline__ void load_window(uint32_t (&av)[NP][NP], __amdgpu_buffer_rsrc_t rs,
                                            const uint32_t (&vo)[NP][NP], uint32_t soff) {
#pragma unroll
  for (int i = 0; i < NP; ++i)
#pragma unroll
    for (int k = 0; k < NP; ++k) av[i][k] = ld_u32(rs, vo[i][k], soff);
}

// Sum one input segment (cw words per pixel) into D, one word's window at
// a time: the waves of a launch overlap each other's load latency (measured
// faster than keeping further words in flight in each wave, which costs
// registers and, for one-word inputs, wasted loads).
template <int MT, int COG>
__device__ __forceinline__ void conv_segment(Acc<MT, COG>& D, __amdgpu_buffer_rsrc_t rs,
                                             const uint32_t (&vo)[MT + 2][MT + 2],
                                             const uint32_t (&m)[MT + 2][MT + 2], int cw,
                                             const uint32_t* __restrict__ wt, int rowstride) {
  constexpr int NP = MT + 2;
  uint32_t win[NP][NP];
#pragma unroll 1
  for (int w = 0; w < cw; ++w) {
    load_window<NP>(win, rs, vo, (uint32_t)w * 4u);
    accumulate<MT, COG>(D, win, m, wt + (size_t)w * rowstride);
  }
}

// Store the COG bits of one channel group.  A group that alone covers its
// 32-bit word writes the whole word; otherwise the last group also writes 0
// to the bytes above it (at most 3), so every word is fully written even
// when cout is not a multiple of 32.
template <int COG>
__device__ __forceinline__ void store_bits(uint32_t* base, size_t pix, int cw, int co0, int cout, uint32_t bits,
                                           int zero_end) {
  uint8_t* row = reinterpret_cast<uint8_t*>(base) + pix * (size_t)cw * 4;
  uint8_t* dst = row + (co0 >> 3);
  if (COG == 32 || ((co0 & 31) == 0 && co0 + COG >= cout)) {
    *reinterpret_cast<uint32_t*>(dst) = bits;
    return;
  }
  if (COG == 16) *reinterpret_cast<uint16_t*>(dst) = (uint16_t)bits;
  else *dst = (uint8_t)bits;
  for (int b = (co0 + COG) >> 3; b < zero_end; ++b) row[b] = 0;
}

// The 1x1 head of one pixel: per class the bias, then the channels in
// order, one fused step each (csrc/bnn_head.c:21-34,
// csrc/bnn_react_opt.c:33-41).  The weights come through the constant
// address space (scalar loads that the logits stores cannot invalidate).
// When the group holds exactly cout channels the weights of a class are
// fetched as one batch, one wait per class instead of one per weight; the
// guarded loop serves a smaller cout.
template <int COG>
__device__ __forceinline__ void head_logits(const float* hw_, const float* hb_, int ncls, int cout,
                                            const float (&v)[COG], float* logits, size_t lbase, size_t lstride) {
  typedef const __attribute__((address_space(4))) float* const_hf;
  const const_hf hw = (const_hf)hw_, hb = (const_hf)hb_;
  if (cout == COG) {
#pragma unroll 1
    for (int o = 0; o < ncls; ++o) {
      float w[COG];
#pragma unroll
      for (int j = 0; j < COG; ++j) w[j] = hw[o * COG + j];
      float accf = hb[o];
#pragma unroll
      for (int j = 0; j < COG; ++j) accf = __fmaf_rn(w[j], v[j], accf);
      logits[lbase + (size_t)o * lstride] = accf;
    }
    return;
  }
#pragma unroll 1
  for (int o = 0; o < ncls; ++o) {
    float accf = hb[o];
#pragma unroll
    for (int j = 0; j < COG; ++j)
      if (j < cout) accf = __fmaf_rn(hw[o * cout + j], v[j], accf);
    logits[lbase + (size_t)o * lstride] = accf;
  }
}

template <int MT, int COG, int EPI, bool DUMP>
__global__ __launch_bounds__(kBlock) void k_bconv(const BconvArgs a, uint32_t bytes0, uint32_t bytes1) {
  constexpr int NP = MT + 2;
  // Block order.  Plain: group g of tile block t is block g * ntb + t.
  // XCD-aware (a.xorder, for outputs in two or more channel groups):
  // consecutive blocks go to the 8 XCDs in turn, so block b runs on XCD
  // b % 8, and its index j = b / 8 there walks (tile block, channel group)
  // with the group fastest, tile block (j / ngroups) * 8 + b % 8.  Every
  // group of a tile block then runs on one XCD, one after the other, and
  // the pieces of a pixel's output words they write merge in that XCD's L2:
  // in the plain order they left L2 as separate partial writes, 8x the
  // output bytes for 128 channels in groups of 16, and 2x for one word per
  // pixel in two groups (config 4's enc1.c2: the same time in either order,
  // as are the v1 and v3 forwards).  (Tile blocks are padded to a multiple
  // of 8; a tile past the end is inactive.)
  const uint32_t ngroups = (uint32_t)(a.cout + COG - 1) / COG;
  uint32_t gidx, tile;
  if (a.xorder) {
    const uint32_t xj = blockIdx.x >> 3;
    gidx = xj % ngroups;
    tile = ((xj / ngroups) * 8u + (blockIdx.x & 7u)) * kBlock + threadIdx.x;
  } else if (ngroups == 1) {
    gidx = 0;
    tile = blockIdx.x * kBlock + threadIdx.x;
  } else {
    const uint32_t ntb = (a.ntiles + kBlock - 1) / kBlock;
    gidx = blockIdx.x / ntb;
    tile = (blockIdx.x - gidx * ntb) * kBlock + threadIdx.x;
  }
  const bool active = tile < a.ntiles;
  if (!active) tile = a.ntiles - 1;
  const uint32_t n = fdiv(tile, a.dper);
  const uint32_t rr = tile - n * a.dper.d;
  const uint32_t ty = fdiv(rr, a.dtw);
  const uint32_t tx = rr - ty * a.dtw.d;
  const int y0 = (int)ty * MT, x0 = (int)tx * MT;
  const int co0 = (int)gidx * COG;
  const int coutp = (a.cout + 31) & ~31;  // weight rows are padded to 32

  // The (MT+2)^2 window around the tile: a row or column outside the image
  // gets a zero mask and is read from the tile's own first row or column,
  // so every load stays inside the tensor.
  bool rok[NP], cok[NP];
  int rc[NP], cc[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int iy = y0 - 1 + i, ix = x0 - 1 + i;
    rok[i] = (uint32_t)iy < (uint32_t)a.H;
    cok[i] = (uint32_t)ix < (uint32_t)a.W;
    rc[i] = rok[i] ? iy : y0;
    cc[i] = cok[i] ? ix : x0;
  }
  uint32_t m[NP][NP], vo[NP][NP];
  {
    const uint32_t cw4 = (uint32_t)a.cw0 * 4u;
    uint32_t ro[NP], co[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      ro[i] = (n * (uint32_t)a.H + (uint32_t)rc[i]) * (uint32_t)a.W * cw4;
      co[i] = (uint32_t)cc[i] * cw4;
    }
#pragma unroll
    for (int i = 0; i < NP; ++i)
#pragma unroll
      for (int k = 0; k < NP; ++k) {
        m[i][k] = (rok[i] && cok[k]) ? ~0u : 0u;
        vo[i][k] = ro[i] + co[k];
      }
  }

  Acc<MT, COG> D;
#pragma unroll
  for (int p = 0; p < MT * MT; ++p)
#pragma unroll
    for (int j = 0; j < COG; ++j) D.d[p][j] = 0;

  if (a.pair) {
    uint32_t win[NP][NP];
    load_window<NP>(win, make_rsrc(a.in0, bytes0), vo, 0u);
    accumulate_pair<MT, COG>(D, win, m, a.wt + (size_t)co0 * 5);
  } else {
    conv_segment<MT, COG>(D, make_rsrc(a.in0, bytes0), vo, m, a.cw0, a.wt + (size_t)co0 * 9, coutp * 9);
  }
  if (a.cw1 > 0) {
    // nearest 2x of the low-res tensor placed at (oh, ow); in-image positions
    // it does not cover read at padoff: v1, past the end of the buffer, where
    // buffer loads return 0 bits (the reference's zero-filled concat, whose 0
    // entries its XNOR kernels treat as -1: csrc/bnn_model.c:130-148,
    // csrc/bnn_conv.c:123, 162); v3, the pad pixel holding the tap bits of
    // the concat's 0.0 (csrc/bnn_model_react.c:280-298).
    const uint32_t cw4 = (uint32_t)a.cw1 * 4u;
    uint32_t lr[NP], lc[NP];
    bool rcov[NP], ccov[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int uy = rc[i] - a.oh, ux = cc[i] - a.ow;
      rcov[i] = (uint32_t)uy < (uint32_t)a.uh;
      ccov[i] = (uint32_t)ux < (uint32_t)a.uw;
      lr[i] = (n * (uint32_t)a.h1 + (uint32_t)(rcov[i] ? uy >> 1 : 0)) * (uint32_t)a.w1 * cw4;
      lc[i] = (uint32_t)(ccov[i] ? ux >> 1 : 0) * cw4;
    }
#pragma unroll
    for (int i = 0; i < NP; ++i)
#pragma unroll
      for (int k = 0; k < NP; ++k) vo[i][k] = (rcov[i] && ccov[k]) ? lr[i] + lc[k] : a.padoff;
    // (after the first segment's table: 9 words per channel and word, or
    // 5 per channel when that segment takes paired taps)
    const size_t seg1 = a.pair ? (size_t)coutp * 5 + (size_t)co0 * 9 : ((size_t)a.cw0 * coutp + co0) * 9;
    conv_segment<MT, COG>(D, make_rsrc(a.in1, bytes1), vo, m, a.cw1, a.wt + seg1, coutp * 9);
  }
  if (!active) return;

  // ---------------------------------------------------------- epilogue --
  int32_t nvalid[MT * MT];
  bool inimg[MT * MT];
#pragma unroll
  for (int py = 0; py < MT; ++py)
#pragma unroll
    for (int px = 0; px < MT; ++px) {
      inimg[py * MT + px] = y0 + py < a.H && x0 + px < a.W;
      const int nr = (int)rok[py] + (int)rok[py + 1] + (int)rok[py + 2];
      const int nc = (int)cok[px] + (int)cok[px + 1] + (int)cok[px + 2];
      nvalid[py * MT + px] = nr * nc * a.cin;
    }
  auto Pof = [&](int p, int j) -> int32_t { return nvalid[p] - 2 * (int32_t)D.d[p][j]; };

  const int HW = a.H * a.W;
  if (EPI == EPI_P || DUMP) {
#pragma unroll
    for (int py = 0; py < MT; ++py)
#pragma unroll
      for (int px = 0; px < MT; ++px) {
        if (!inimg[py * MT + px]) continue;
        const int pix = (y0 + py) * a.W + x0 + px;
#pragma unroll
        for (int j = 0; j < COG; ++j)
          if (co0 + j < a.cout) a.P[((size_t)n * a.cout + co0 + j) * HW + pix] = Pof(py * MT + px, j);
      }
  }
  if (EPI == EPI_P) return;

  // bytes of the pixel's words the last channel group zero-fills
  const int zero_end = gidx == ngroups - 1 ? a.cwo * 4 : 0;

  if constexpr (EPI == EPI_RX || EPI == EPI_RXPOOL || EPI == EPI_RXHEAD) {
    // h = RPReLU(fma(A, P, B + move1) + res): the fused step and the two
    // separately rounded operations of csrc/bnn_react_epi.c:34-55 as the
    // reference build contracts them; tap bit = h + rsign > 0
    // (csrc/bnn_react_ops.c:75-85)
    const size_t plane = (size_t)(a.ntot ? a.ntot : a.N) * HW;  // positions per plane
    // the per-channel parameters through the constant address space: the
    // kernel never writes them, and saying so makes their loads scalar
    typedef const __attribute__((address_space(4))) float* const_f32;
    const const_f32 eA = (const_f32)a.eA + co0, eB = (const_f32)a.eB + co0, eW = (const_f32)a.eW + co0;
    const const_f32 trs = a.trs ? (const_f32)a.trs + co0 : nullptr;
    // one scalar descriptor per channel plane of `base`, size 0 past cout:
    // loads there read 0 and stores are dropped
    auto plane_rsrc = [&](const float* base, int j, size_t psize) {
      const bool cok = co0 + j < a.cout;
      const uint64_t b = (uint64_t)(uintptr_t)base + (uint64_t)(cok ? co0 + j : 0) * psize * 4;
      const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
      const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
      const uint32_t bytes = (uint32_t)__builtin_amdgcn_readfirstlane((int)(cok ? (uint32_t)psize * 4u : 0u));
      return make_rsrc((const void*)(uintptr_t)(((uint64_t)hi << 32) | lo), bytes);
    };
    auto rx = [](int32_t P, float A, float Bm, float w, float res) {
      const float t = __fadd_rn(__fmaf_rn(A, (float)P, Bm), res);
      return t >= 0.0f ? t : __fmul_rn(w, t);
    };
    constexpr int JP = COG < 8 ? COG : 8;  // channels per parameter batch
    float hr[MT * MT][COG];  // the shortcut at each pixel (EPI_RXPOOL pools it)
    uint32_t bits[MT * MT];
#pragma unroll
    for (int p = 0; p < MT * MT; ++p) bits[p] = 0;
    // a 2x2 block's two pixels of a row move as one 8-byte access when the
    // width is even (then both lie inside the image or neither does)
    const bool pairs = MT == 2 && (a.W & 1) == 0;
    // every shortcut value is loaded before the first store: the stores may
    // alias them as far as the compiler knows, and interleaved they would
    // wait for one load at a time
    if (pairs) {
#pragma unroll
      for (int py = 0; py < MT; ++py) {
        const size_t pix = ((size_t)n * a.H + y0 + py) * a.W + x0;
        const uint32_t voff = inimg[py * MT] ? (uint32_t)pix * 4u : 0x80000000u;
#pragma unroll
        for (int j = 0; j < COG; ++j) {
          const stem_f32x2 v = raw_load_f32x2(plane_rsrc(a.res, j, plane), (int)voff, 0, 0);
          hr[py * MT][j] = v[0];
          hr[py * MT + 1][j] = v[1];
        }
      }
    } else {
#pragma unroll
      for (int py = 0; py < MT; ++py)
#pragma unroll
        for (int px = 0; px < MT; ++px) {
          const int p = py * MT + px;
          const size_t pix = ((size_t)n * a.H + y0 + py) * a.W + x0 + px;
          // one descriptor per channel plane (a channel past cout gets size
          // 0), the pixel's offset past the end when it lies outside the image
          const uint32_t voff = inimg[p] ? (uint32_t)pix * 4u : 0x80000000u;
#pragma unroll
          for (int j = 0; j < COG; ++j) hr[p][j] = ld_f32(plane_rsrc(a.res, j, plane), voff, 0);
        }
    }
#pragma unroll
    for (int py = 0; py < MT; ++py) {
      const size_t row = ((size_t)n * a.H + y0 + py) * a.W + x0;
      // no branches: a pixel outside the image stores past the end (dropped)
      // and a channel past cout into a zero-sized plane; neither sets a bit
      uint32_t voff[MT];
#pragma unroll
      for (int px = 0; px < MT; ++px) voff[px] = inimg[py * MT + px] ? (uint32_t)(row + px) * 4u : 0x80000000u;
      // the parameters of JP channels in one batch of scalar loads (next to
      // their uses, after the stores of the previous channel, each would be
      // waited for alone); the tap rsign index stays below cout
#pragma unroll
      for (int j0 = 0; j0 < COG; j0 += JP) {
        float pA[JP], pB[JP], pW[JP], pT[JP];
#pragma unroll
        for (int jj = 0; jj < JP; ++jj) {
          pA[jj] = eA[j0 + jj];
          pB[jj] = eB[j0 + jj];
          pW[jj] = eW[j0 + jj];
          pT[jj] = trs ? trs[min(co0 + j0 + jj, a.cout - 1) - co0] : 0.0f;
        }
#pragma unroll
        for (int jj = 0; jj < JP; ++jj) {
          const int j = j0 + jj;
          float h[MT];
#pragma unroll
          for (int px = 0; px < MT; ++px) {
            const int p = py * MT + px;
            h[px] = rx(Pof(p, j), pA[jj], pB[jj], pW[jj], hr[p][j]);
            if (trs && co0 + j < a.cout && __fadd_rn(h[px], pT[jj]) > 0.0f) bits[p] |= 1u << j;
            if constexpr (EPI == EPI_RXHEAD) hr[p][j] = h[px];
          }
          if (a.hout) {
            const __amdgpu_buffer_rsrc_t hd = plane_rsrc(a.hout, j, plane);
            if constexpr (MT == 2) {
              if (pairs) {
                raw_store_f32x2(stem_f32x2{h[0], h[1]}, hd, (int)voff[0], 0, 0);
                continue;
              }
            }
#pragma unroll
            for (int px = 0; px < MT; ++px)
              __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, h[px]), hd, (int)voff[px], 0, 0);
          }
        }
      }
#pragma unroll
      for (int px = 0; px < MT; ++px)
        if (trs && a.out && inimg[py * MT + px])
          store_bits<COG>(a.out, row + px, a.cwo, co0, a.cout, bits[py * MT + px], zero_end);
    }
    // the pad pixel after the last one of the whole batch: the tap bits of
    // 0.0, read by a concat where its upsample does not cover
    // (csrc/bnn_model_react.c:282)
    if (EPI == EPI_RX && trs && a.out && tile == 0 && threadIdx.x == 0) {
      uint32_t pb = 0;
#pragma unroll
      for (int j = 0; j < COG; ++j)
        if (co0 + j < a.cout && __fadd_rn(0.0f, trs[j]) > 0.0f) pb |= 1u << j;
      store_bits<COG>(a.out, plane - (size_t)a.n0 * HW, a.cwo, co0, a.cout, pb, zero_end);
    }
    if constexpr (EPI == EPI_RXPOOL) {
      // 2x2 floor-mode max of P (csrc/bnn_react_opt.c:71-82) and of the
      // highway read (0,0), (0,1), (1,0), (1,1), first of equals kept
      // (csrc/bnn_react_opt.c:61-66); then the down epilogue on both
      const bool pooled = y0 + 1 < a.H && x0 + 1 < a.W;
      if (!pooled) return;
      const int Hh = a.H >> 1, Wh = a.W >> 1;
      const size_t hplane = (size_t)(a.ntot ? a.ntot : a.N) * Hh * Wh, dp = ((size_t)n * Hh + ty) * Wh + tx;
      const const_f32 drs = a.drs ? (const_f32)a.drs + co0 : nullptr;
      uint32_t b2 = 0;
#pragma unroll
      for (int j0 = 0; j0 < COG; j0 += JP) {
        // one batch of scalar loads per JP channels, indices kept below cout
        float qA[JP], qB[JP], qW[JP], qT[JP];
#pragma unroll
        for (int jj = 0; jj < JP; ++jj) {
          const int c = min(co0 + j0 + jj, a.cout - 1);
          qA[jj] = ((const_f32)a.dA)[c];
          qB[jj] = ((const_f32)a.dB)[c];
          qW[jj] = ((const_f32)a.dW)[c];
          qT[jj] = drs ? drs[c - co0] : 0.0f;
        }
#pragma unroll
        for (int jj = 0; jj < JP; ++jj) {
          const int j = j0 + jj;
          if (co0 + j >= a.cout) continue;
          int32_t pm = Pof(0, j);
          float hm = hr[0][j];
#pragma unroll
          for (int p = 1; p < 4; ++p) {
            pm = max(pm, Pof(p, j));
            if (hr[p][j] > hm) hm = hr[p][j];
          }
          if (DUMP) a.P2[((size_t)n * a.cout + co0 + j) * Hh * Wh + ty * Wh + tx] = pm;
          const float d = rx(pm, qA[jj], qB[jj], qW[jj], hm);
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, d), plane_rsrc(a.dout, j, hplane),
                                                (int)((uint32_t)dp * 4u), 0, 0);
          if (drs && __fadd_rn(d, qT[jj]) > 0.0f) b2 |= 1u << j;
        }
      }
      if (drs && a.out2) store_bits<COG>(a.out2, dp, a.cwo, co0, a.cout, b2, zero_end);
    }
    if constexpr (EPI == EPI_RXHEAD) {
      // bias, then channels in order, one fused step each
      // (csrc/bnn_react_opt.c:33-41); one group holds every channel
      const int pix = y0 * a.W + x0;
      size_t lbase = (size_t)n * a.ncls * HW + pix, lstride = HW;
      if (a.pcols > 0) {
        const int pr = a.prow0 + (int)n / a.pcols, pc = (int)n % a.pcols;
        const int sy = pr * a.H + y0, sx = pc * a.W + x0;
        if (sy >= a.sH || sx >= a.sW) return;
        lbase = (size_t)sy * a.sW + sx;
        lstride = (size_t)a.sH * a.sW;
      }
      head_logits<COG>(a.hw, a.hb, a.ncls, a.cout, hr[0], a.logits, lbase, lstride);
    }
    return;
  }
  const int32_t* lo1 = a.f1.lo + co0;
  const uint32_t* wd1 = a.f1.wid + co0;
  uint32_t bits[MT * MT];
#pragma unroll
  for (int p = 0; p < MT * MT; ++p) bits[p] = 0;

  if (EPI == EPI_POOL) {
    // rule 1 on each P, 2x2 floor-mode max of P (csrc/bnn_maxpool.c:28-48),
    // then rule 2 on the max
    const int32_t* lo2 = a.f2.lo + co0;
    const uint32_t* wd2 = a.f2.wid + co0;
    const bool pooled = y0 + 1 < a.H && x0 + 1 < a.W;
    const int Hh = a.H >> 1, Wh = a.W >> 1;
    uint32_t b2 = 0;
#pragma unroll
    for (int j = 0; j < COG; ++j) {
      int32_t pm = INT32_MIN;
#pragma unroll
      for (int p = 0; p < MT * MT; ++p) {
        const int32_t P = Pof(p, j);
        bits[p] |= ((uint32_t)P - (uint32_t)lo1[j] < wd1[j] ? 1u : 0u) << j;
        pm = max(pm, P);
      }
      b2 |= ((uint32_t)pm - (uint32_t)lo2[j] < wd2[j] ? 1u : 0u) << j;
      if (DUMP && pooled && co0 + j < a.cout)
        a.P2[((size_t)n * a.cout + co0 + j) * Hh * Wh + ty * Wh + tx] = pm;
    }
    if (a.out != nullptr) {
#pragma unroll
      for (int py = 0; py < MT; ++py)
#pragma unroll
        for (int px = 0; px < MT; ++px)
          if (inimg[py * MT + px])
            store_bits<COG>(a.out, ((size_t)n * a.H + y0 + py) * a.W + x0 + px, a.cwo, co0, a.cout,
                            bits[py * MT + px], zero_end);
    }
    if (pooled) store_bits<COG>(a.out2, ((size_t)n * Hh + ty) * Wh + tx, a.cwo, co0, a.cout, b2, zero_end);
    return;
  }

  if (EPI == EPI_FOLD) {
#pragma unroll
    for (int j = 0; j < COG; ++j)
#pragma unroll
      for (int p = 0; p < MT * MT; ++p) bits[p] |= ((uint32_t)Pof(p, j) - (uint32_t)lo1[j] < wd1[j] ? 1u : 0u) << j;
#pragma unroll
    for (int py = 0; py < MT; ++py)
#pragma unroll
      for (int px = 0; px < MT; ++px)
        if (inimg[py * MT + px])
          store_bits<COG>(a.out, ((size_t)n * a.H + y0 + py) * a.W + x0 + px, a.cwo, co0, a.cout,
                          bits[py * MT + px], zero_end);
    return;
  }

  if (EPI == EPI_HEAD) {
    // rule, widen to +-1 and the 1x1 head: bias first, then channels in
    // order, one fused step each (csrc/bnn_head.c:21-34).  One group holds
    // every channel (cout <= COG).
    float sg[COG];
#pragma unroll
    for (int j = 0; j < COG; ++j) {
      const bool b = (uint32_t)Pof(0, j) - (uint32_t)lo1[j] < wd1[j];
      bits[0] |= (b ? 1u : 0u) << j;
      sg[j] = b ? 1.0f : -1.0f;
    }
    if (a.out) store_bits<COG>(a.out, ((size_t)n * a.H + y0) * a.W + x0, a.cwo, co0, a.cout, bits[0], zero_end);
    const int pix = y0 * a.W + x0;
    // batch: logits [N][ncls][H][W]; scene: the map [ncls][sH][sW], pixels
    // of an edge patch past the scene dropped
    size_t lbase = (size_t)n * a.ncls * HW + pix, lstride = HW;
    bool keep = true;
    if (a.pcols > 0) {
      const int pr = a.prow0 + (int)n / a.pcols, pc = (int)n % a.pcols;
      const int sy = pr * a.H + y0, sx = pc * a.W + x0;
      keep = sy < a.sH && sx < a.sW;
      lbase = (size_t)sy * a.sW + sx;
      lstride = (size_t)a.sH * a.sW;
    }
    if (!keep) return;
    head_logits<COG>(a.hw, a.hb, a.ncls, a.cout, sg, a.logits, lbase, lstride);
  }
}

// ------------------------------------------------------------------------
// v3 1x1 projection (real weights, no bias) on the matrix cores
// ------------------------------------------------------------------------
// out[co][q] = chain over ci from 0 of fma(W[co][ci], x[ci][q], acc) from +0
// (csrc/bnn_realin_blk.h:59-70): each K = 1 MFMA step is that fma, exactly.
// A wave owns 64 consecutive plane positions q0 + l (B block l/16, column
// l%16) and G groups of 16 output channels.  Per four input channels one
// A register per group holds their weights (lanes 16k + i = W[16g + i][4c + k],
// block k broadcast by CBSZ = 2, ABID = k).  The concat of a decoder reads
// channels past c0 from the nearest-2x upsample of x1; positions it does not
// cover, and channels past cin, read 0, which leaves the chain unchanged
// (w*0 is +-0 and the chain never holds -0).
template <int G, int K>
__device__ __forceinline__ void proj_step(f32x16 (&acc)[G], const float (&wa)[G], const float (&xb)[4]) {
#pragma unroll
  for (int gi = 0; gi < G; ++gi) acc[gi] = __builtin_amdgcn_mfma_f32_16x16x1f32(wa[gi], xb[K], acc[gi], 2, K, 0);
}
template <int G, int... K>
__device__ __forceinline__ void proj_steps(f32x16 (&acc)[G], const float (&wa)[G], const float (&xb)[4],
                                           std::integer_sequence<int, K...>) {
  (proj_step<G, K>(acc, wa, xb), ...);
}

// what a wave of k_proj needs to fetch its inputs: one descriptor per
// source (the planes of x0, and of x1 for a concat), a channel selected by
// the scalar offset, the lane's position by the vector offset (0x80000000,
// past every source, for a lane with nothing to read)
struct ProjSrc {
  __amdgpu_buffer_rsrc_t w, r0, r1;
  uint32_t nq4, pl4;          // bytes per plane of x0 / x1
  uint32_t voff0, voff1;
  int nquad, g0, lane;
};

// U quads of one source: G weight registers and 4 inputs per quad, the
// inputs of quad c4 at scalar offset so + (4*(c4 - qa) + k) * step.  The
// offsets advance by additions only (the scalar unit is shared by the CU).
template <int G, int U>
__device__ __forceinline__ void proj_load(const ProjSrc& S, __amdgpu_buffer_rsrc_t rs, uint32_t vo, uint32_t so,
                                          uint32_t step, int c4, float (&wa)[U][G], float (&xb)[U][4]) {
  uint32_t wso = (uint32_t)((S.g0 * S.nquad + c4) * 256);
#pragma unroll
  for (int u = 0; u < U; ++u, wso += 256) {
    uint32_t g = wso;
#pragma unroll
    for (int gi = 0; gi < G; ++gi, g += (uint32_t)S.nquad * 256u) wa[u][gi] = ld_f32(S.w, (uint32_t)S.lane * 4u, g);
#pragma unroll
    for (int k = 0; k < 4; ++k, so += step) xb[u][k] = ld_f32(rs, vo, so);
  }
}

// the chain steps of one batch; quads at or past qb are skipped (uniform)
template <int G, int U>
__device__ __forceinline__ void proj_run(f32x16 (&acc)[G], const float (&wa)[U][G], const float (&xb)[U][4], int c4,
                                         int qb) {
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (c4 + u < qb) proj_steps<G>(acc, wa[u], xb[u], std::make_integer_sequence<int, 4>{});
}

// quads [qa, qb) of one source, batch b+1 fetched while batch b runs: each
// output is one chain of cin dependent steps, so a wave's loads must
// overlap its products
template <int G, int U>
__device__ __forceinline__ void proj_range(f32x16 (&acc)[G], const ProjSrc& S, __amdgpu_buffer_rsrc_t rs, uint32_t vo,
                                           uint32_t so, uint32_t step, int qa, int qb) {
  if (qa >= qb) return;
  const uint32_t bstep = step * 4u * U;
  float wa0[U][G], xb0[U][4], wa1[U][G], xb1[U][4];
  proj_load<G, U>(S, rs, vo, so, step, qa, wa0, xb0);
#pragma unroll 1
  for (int c4 = qa; c4 < qb; c4 += 2 * U) {
    so += bstep;
    if (c4 + U < qb) proj_load<G, U>(S, rs, vo, so, step, c4 + U, wa1, xb1);
    proj_run<G, U>(acc, wa0, xb0, c4, qb);
    if (c4 + U >= qb) break;
    so += bstep;
    if (c4 + 2 * U < qb) proj_load<G, U>(S, rs, vo, so, step, c4 + 2 * U, wa0, xb0);
    proj_run<G, U>(acc, wa1, xb1, c4 + U, qb);
  }
}

template <int G>
__global__ __launch_bounds__(256) void k_proj(const ProjArgs a) {
  constexpr int U = G <= 2 ? 8 : 4;  // quads per batch (two batches of registers)
  const int lane = threadIdx.x & 63;
  // nq positions to process, sq positions per plane (a batch part: its own
  // patches out of ntot)
  const long HW = (long)a.H * a.W, nq = (long)a.N * HW, sq = (long)(a.ntot ? a.ntot : a.N) * HW;
  const long nrel = (long)(a.ntot ? a.ntot - a.n0 : a.N);  // patches from this call's first to the end
  const long q0 = ((long)blockIdx.x * 4 + (threadIdx.x >> 6)) * 64;
  if (q0 >= nq) return;  // whole waves
  const long q = q0 + lane;
  const bool qok = q < nq;
  const int ngrp = (a.cout + 15) / 16, nquad = (a.cin + 3) / 4;
  constexpr uint32_t kFar = 0x80000000u;  // plane sets stay below 2 GiB (launch_proj checks)
  ProjSrc S;
  const uint32_t plane1 = (uint32_t)((size_t)(a.ntot ? a.ntot : a.N) * a.h1 * a.w1);
  S.w = make_rsrc(a.w, (uint32_t)((size_t)ngrp * nquad * 256));
  // each source from this call's first position to the end of its last plane
  S.r0 = make_rsrc(a.x0, a.c0 ? (uint32_t)(((size_t)(a.c0 - 1) * sq + nrel * HW) * 4) : 0u);
  S.r1 = make_rsrc(a.x1 ? a.x1 : a.x0,
                   a.x1 ? (uint32_t)(((size_t)(a.cin - a.c0 - 1) * plane1 + nrel * a.h1 * a.w1) * 4) : 0u);
  S.nq4 = (uint32_t)sq * 4u;
  S.pl4 = plane1 * 4u;
  S.voff0 = qok ? (uint32_t)q * 4u : kFar;
  S.voff1 = kFar;
  if (a.x1 && qok) {
    const long n = q / HW, rem = q - n * HW;
    const int y = (int)(rem / a.W), x = (int)(rem - (long)y * a.W);
    const int uy = y - a.oh, ux = x - a.ow;
    if ((unsigned)uy < (unsigned)a.uh && (unsigned)ux < (unsigned)a.uw)
      S.voff1 = (uint32_t)(((size_t)n * a.h1 + (uy >> 1)) * a.w1 + (ux >> 1)) * 4u;
  }
  S.nquad = nquad; S.g0 = blockIdx.y * G; S.lane = lane;
  f32x16 acc[G];
#pragma unroll
  for (int gi = 0; gi < G; ++gi)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[gi][r] = 0.0f;
  // input channels in order: the quads wholly in x0, the one quad that
  // crosses into x1 (when c0 is not a multiple of 4), the quads of x1.
  // Channels past cin lie past their source and read 0.
  if (!a.x1) {
    proj_range<G, U>(acc, S, S.r0, S.voff0, 0u, S.nq4, 0, nquad);
  } else {
    const int qx = a.c0 / 4;
    proj_range<G, U>(acc, S, S.r0, S.voff0, 0u, S.nq4, 0, qx);
    if (a.c0 % 4) {
      float wa[1][G], xb[1][4];
      proj_load<G, 1>(S, S.r0, S.voff0, (uint32_t)(4 * qx) * S.nq4, S.nq4, qx, wa, xb);
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (4 * qx + k >= a.c0) xb[0][k] = ld_f32(S.r1, S.voff1, (uint32_t)(4 * qx + k - a.c0) * S.pl4);
      proj_run<G, 1>(acc, wa, xb, qx, nquad);
    }
    const int qa = (a.c0 + 3) / 4;
    proj_range<G, U>(acc, S, S.r1, S.voff1, (uint32_t)(4 * qa - a.c0) * S.pl4, S.pl4, qa, nquad);
  }
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int co = 16 * (S.g0 + gi) + 4 * (lane >> 4) + (r & 3);
      const long qq = q0 + 16 * (r >> 2) + (lane & 15);
      if (co < a.cout && qq < nq) a.out[(size_t)co * sq + qq] = acc[gi][r];
    }
  }
}

// ------------------------------------------------------------------------
// simple kernels for the v3 batch-1 kernel ABI
// ------------------------------------------------------------------------
// t = A*acc + B + res + move1 (form 0: csrc/bnn_react_ops.c:47, contracted to
// fma(A, acc, B) then two adds) or A*acc + (B + move1) + res (form 1:
// csrc/bnn_react_epi.c:30,53,75, fma(A, acc, B + move1) then one add);
// out = t >= 0 ? t : prelu_w * t.  acc: 0 int32, 1 int16, 2 float.
__global__ void k_react_epi(const void* __restrict__ acc, int kind, const float* __restrict__ res,
                            float* __restrict__ out, int C, long HW, const float* __restrict__ A,
                            const float* __restrict__ B, const float* __restrict__ m,
                            const float* __restrict__ w, int form) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)C * HW) return;
  const int c = (int)(i / HW);
  const float v = kind == 0 ? (float)((const int32_t*)acc)[i]
                  : kind == 1 ? (float)((const int16_t*)acc)[i]
                              : ((const float*)acc)[i];
  float t;
  if (form == 0) t = __fadd_rn(__fadd_rn(__fmaf_rn(A[c], v, B[c]), res[i]), m[c]);
  else t = __fadd_rn(__fmaf_rn(A[c], v, __fadd_rn(B[c], m[c])), res[i]);
  out[i] = t >= 0.0f ? t : __fmul_rn(w[c], t);
}

// sign(x + rsign) as +-1 (csrc/bnn_react_ops.c:75-85)
__global__ void k_react_tap(const float* __restrict__ x, int8_t* __restrict__ out, int C, long HW,
                            const float* __restrict__ rsign) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)C * HW) return;
  out[i] = __fadd_rn(x[i], rsign[i / HW]) > 0.0f ? 1 : -1;
}

// k x k / stride max from -inf, window row-major, first of equals kept
// (csrc/bnn_react_ops.c:89-107)
__global__ void k_maxpool_real(const float* __restrict__ x, float* __restrict__ out, int C, int H, int W, int k,
                               int stride) {
  const int Ho = (H - k) / stride + 1, Wo = (W - k) / stride + 1;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)C * Ho * Wo) return;
  const int c = (int)(i / ((long)Ho * Wo)), r = (int)(i % ((long)Ho * Wo)), oy = r / Wo, ox = r % Wo;
  float mx = -__builtin_inff();
  for (int ky = 0; ky < k; ++ky)
    for (int kx = 0; kx < k; ++kx) {
      const float v = x[((size_t)c * H + oy * stride + ky) * W + ox * stride + kx];
      if (v > mx) mx = v;
    }
  out[i] = mx;
}

// 3x3 / pad 1 / stride 1, +-1 (or any int8) weights: per output one chain,
// input channels outermost, taps row-major inside, taps outside the image
// skipped, then alpha * acc (csrc/bnn_realin_blk.h:111-147)
__global__ void k_conv3_chain(const float* __restrict__ x, const int8_t* __restrict__ wsign,
                              const float* __restrict__ alpha, float* __restrict__ out, int cin, int H, int W,
                              int cout) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)cout * H * W) return;
  const int co = (int)(i / ((long)H * W)), r = (int)(i % ((long)H * W)), oy = r / W, ox = r % W;
  float acc = 0.0f;
  for (int ci = 0; ci < cin; ++ci)
    for (int ky = 0; ky < 3; ++ky) {
      const int iy = oy + ky - 1;
      if (iy < 0 || iy >= H) continue;
      for (int kx = 0; kx < 3; ++kx) {
        const int ix = ox + kx - 1;
        if (ix < 0 || ix >= W) continue;
        acc = __fmaf_rn((float)wsign[((size_t)co * cin + ci) * 9 + ky * 3 + kx],
                        x[((size_t)ci * H + iy) * W + ix], acc);
      }
    }
  out[i] = __fmul_rn(alpha[co], acc);
}

// ------------------------------------------------------------------------
// simple kernels for the batch-1 kernel ABI
// ------------------------------------------------------------------------
// int8 [N][C][H][W] (value > 0 -> bit 1) -> uint32 [N][H][W][ceil(C/32)]
__global__ void k_pack_act(const int8_t* __restrict__ a, uint32_t* __restrict__ out, int N, int C, int H, int W) {
  const int cw = (C + 31) >> 5;
  const long HW = (long)H * W;
  const long total = (long)N * HW * cw;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int w = (int)(i % cw);
  const long pix = i / cw;
  const long n = pix / HW, p = pix - n * HW;
  uint32_t word = 0;
  for (int b = 0; b < 32; ++b) {
    const int c = w * 32 + b;
    if (c < C && a[((size_t)n * C + c) * HW + p] > 0) word |= 1u << b;
  }
  out[i] = word;
}

__global__ void k_bconv_generic(const uint32_t* __restrict__ act, const uint32_t* __restrict__ wt,
                                int32_t* __restrict__ P, int cin, int H, int W, int cout, int kh, int kw,
                                int pad, int stride) {
  const int Ho = (H + 2 * pad - kh) / stride + 1, Wo = (W + 2 * pad - kw) / stride + 1;
  const long total = (long)cout * Ho * Wo;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int co = (int)(i / ((long)Ho * Wo));
  const int r = (int)(i - (long)co * Ho * Wo);
  const int oy = r / Wo, ox = r - oy * Wo;
  const int cw = (cin + 31) >> 5, taps = kh * kw;
  int nvalid = 0;
  uint32_t d = 0;
  for (int ky = 0; ky < kh; ++ky) {
    const int iy = oy * stride + ky - pad;
    if (iy < 0 || iy >= H) continue;
    for (int kx = 0; kx < kw; ++kx) {
      const int ix = ox * stride + kx - pad;
      if (ix < 0 || ix >= W) continue;
      nvalid += cin;
      for (int w = 0; w < cw; ++w)
        d += __builtin_popcount(act[((size_t)iy * W + ix) * cw + w] ^ wt[((size_t)w * cout + co) * taps + ky * kw + kx]);
    }
  }
  P[i] = nvalid - 2 * (int32_t)d;
}

__global__ void k_bconv_naive(const int8_t* __restrict__ a, const int8_t* __restrict__ w, int32_t* __restrict__ P,
                              int cin, int H, int W, int cout, int kh, int kw, int pad, int stride) {
  const int Ho = (H + 2 * pad - kh) / stride + 1, Wo = (W + 2 * pad - kw) / stride + 1;
  const long total = (long)cout * Ho * Wo;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int co = (int)(i / ((long)Ho * Wo));
  const int r = (int)(i - (long)co * Ho * Wo);
  const int oy = r / Wo, ox = r - oy * Wo;
  int32_t acc = 0;
  for (int ci = 0; ci < cin; ++ci)
    for (int ky = 0; ky < kh; ++ky) {
      const int iy = oy * stride + ky - pad;
      if (iy < 0 || iy >= H) continue;
      for (int kx = 0; kx < kw; ++kx) {
        const int ix = ox * stride + kx - pad;
        if (ix < 0 || ix >= W) continue;
        acc += (int32_t)w[(((size_t)co * cin + ci) * kh + ky) * kw + kx] * (int32_t)a[((size_t)ci * H + iy) * W + ix];
      }
    }
  P[i] = acc;
}

// general-shape real conv in the reference order; w is float [cout][kh][kw][cin]
__global__ void k_real_generic(const float* __restrict__ x, const float* __restrict__ w,
                               const float* __restrict__ alpha, float* __restrict__ out, int cin, int H,
                               int W, int cout, int kh, int kw, int pad, int stride) {
  const int Ho = (H + 2 * pad - kh) / stride + 1, Wo = (W + 2 * pad - kw) / stride + 1;
  const long total = (long)cout * Ho * Wo;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int co = (int)(i / ((long)Ho * Wo));
  const int r = (int)(i - (long)co * Ho * Wo);
  const int oy = r / Wo, ox = r - oy * Wo;
  const int y0 = oy * stride - pad, x0 = ox * stride - pad;
  const int ky0 = y0 < 0 ? -y0 : 0, ky1 = y0 + kh > H ? H - y0 : kh;
  const int kx0 = x0 < 0 ? -x0 : 0, kx1 = x0 + kw > W ? W - x0 : kw;
  float acc = 0.0f;
  for (int ky = ky0; ky < ky1; ++ky)
    for (int kx = kx0; kx < kx1; ++kx) {
      const float* wv = w + (((size_t)co * kh + ky) * kw + kx) * cin;
      const size_t pix = (size_t)(y0 + ky) * W + (x0 + kx);
      float s = 0.0f;
      for (int ci = 0; ci < cin; ++ci) s = __fadd_rn(s, __fmul_rn(x[(size_t)ci * H * W + pix], wv[ci]));
      acc = __fadd_rn(acc, s);
    }
  out[i] = __fmul_rn(alpha[co], acc);
}

__global__ void k_maxpool(const int32_t* __restrict__ P, int32_t* __restrict__ out, int C, int H, int W, int k,
                          int stride) {
  const int Ho = (H - k) / stride + 1, Wo = (W - k) / stride + 1;
  const long total = (long)C * Ho * Wo;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int c = (int)(i / ((long)Ho * Wo));
  const int r = (int)(i - (long)c * Ho * Wo);
  const int oy = r / Wo, ox = r - oy * Wo;
  int32_t mx = INT32_MIN;
  for (int dy = 0; dy < k; ++dy)
    for (int dx = 0; dx < k; ++dx)
      mx = max(mx, P[((size_t)c * H + oy * stride + dy) * W + ox * stride + dx]);
  out[i] = mx;
}

__global__ void k_fold_int(const int32_t* __restrict__ P, int8_t* __restrict__ out, int C, int HW,
                           const int32_t* __restrict__ type, const int32_t* __restrict__ t,
                           const int32_t* __restrict__ lo, const int32_t* __restrict__ hi) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)C * HW) return;
  const int c = (int)(i / HW);
  const int32_t v = P[i];
  bool on;
  switch (type[c]) {
    case 0: on = t[c] > 0; break;
    case 1: on = v >= t[c]; break;
    case 2: on = v < t[c]; break;
    case 3: on = v >= lo[c] && v < hi[c]; break;
    case 4: on = v < lo[c] || v >= hi[c]; break;
    default: on = false; break;
  }
  out[i] = on ? 1 : -1;
}

__global__ void k_fold_real(const float* __restrict__ x, int8_t* __restrict__ out, int C, int HW,
                            const float* __restrict__ A, const float* __restrict__ B,
                            const float* __restrict__ slope, const float* __restrict__ rsign) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)C * HW) return;
  const int c = (int)(i / HW);
  float z = __fmaf_rn(A[c], x[i], B[c]);
  if (z < 0.0f) z = __fmul_rn(slope[c], z);
  const float r = __fadd_rn(z, rsign[c]);
  out[i] = r > 0.0f ? 1 : -1;
}

__global__ void k_head(const float* __restrict__ a, const float* __restrict__ W, const float* __restrict__ b,
                       float* __restrict__ out, int cin, int HW, int cout) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)cout * HW) return;
  const int o = (int)(i / HW);
  const long p = i - (long)o * HW;
  float acc = b[o];
  for (int c = 0; c < cin; ++c) acc = __fmaf_rn(W[(size_t)o * cin + c], a[(size_t)c * HW + p], acc);
  out[i] = acc;
}

inline unsigned blocks_for(long n, int bs = kBlock) { return (unsigned)((n + bs - 1) / bs); }

// One pixel per lane: per class the bias, then one fused step per input
// channel in order (csrc/bnn_head.c:21-34; csrc/bnn_react_opt.c:23-44, whose
// x86 build contracts lo[p] += w * a[p] to one fma).  The weights come
// through the constant address space (uniform scalar loads).
template <bool BITS>
__global__ __launch_bounds__(kBlock) void k_head_sep(const HeadArgs a) {
  const long i = (long)blockIdx.x * kBlock + threadIdx.x;
  const long HW = (long)a.H * a.W;
  if (i >= (long)a.N * HW) return;
  const int n = (int)(i / HW);
  const long p = i - (long)n * HW;
  const int y = (int)(p / a.W), x = (int)(p - (long)y * a.W);
  size_t lbase = (size_t)n * a.ncls * HW + p, lstride = HW;
  if (a.pcols > 0) {
    const int pr = a.prow0 + n / a.pcols, pc = n % a.pcols;
    const int sy = pr * a.H + y, sx = pc * a.W + x;
    if (sy >= a.sH || sx >= a.sW) return;
    lbase = (size_t)sy * a.sW + sx;
    lstride = (size_t)a.sH * a.sW;
  }
  typedef const __attribute__((address_space(4))) float* const_hf;
  const const_hf hw = (const_hf)a.hw, hb = (const_hf)a.hb;
  const uint32_t* bw = BITS ? a.bits + i * a.cw : nullptr;
#pragma unroll 1
  for (int o = 0; o < a.ncls; ++o) {
    float acc = hb[o];
#pragma unroll 1
    for (int c0 = 0; c0 < a.cin; c0 += 32) {
      const uint32_t word = BITS ? bw[c0 >> 5] : 0u;
      const int cn = min(32, a.cin - c0);
#pragma unroll 4
      for (int k = 0; k < cn; ++k) {
        const float v = BITS ? (((word >> k) & 1u) ? 1.0f : -1.0f) : a.planes[(size_t)(c0 + k) * a.plane + i];
        acc = __fmaf_rn(hw[o * a.cin + c0 + k], v, acc);
      }
    }
    a.logits[lbase + (size_t)o * lstride] = acc;
  }
}

template <int MT, int COG, int EPI, bool DUMP>
hipError_t go_bconv(BconvArgs a, hipStream_t s) {
  const uint32_t tH = (uint32_t)(a.H + MT - 1) / MT, tW = (uint32_t)(a.W + MT - 1) / MT;
  const uint64_t ntiles = (uint64_t)a.N * tH * tW;
  if (ntiles >= 0x80000000ull) return hipErrorInvalidValue;
  a.ntiles = (uint32_t)ntiles;
  a.dper = make_fastdiv(tH * tW);
  a.dtw = make_fastdiv(tW);
  const int groups = (a.cout + COG - 1) / COG;
  const uint32_t b0 = (uint32_t)((size_t)a.N * a.H * a.W * a.cw0 * 4);
  // a pad pixel (v3) lies right after the low-res tensor
  const int nrel = a.ntot ? a.ntot - a.n0 : a.N;  // patches from this call's first to the end
  const uint32_t b1 = a.in1 ? (uint32_t)((size_t)(nrel * a.h1 * a.w1 + (a.padoff != 0x80000000u ? 1 : 0)) *
                                         a.cw1 * 4)
                            : 0u;
  a.xorder = (groups > 1 && EPI != EPI_P) ? 1 : 0;
  const uint64_t nblocks = (uint64_t)(a.xorder ? (blocks_for((long)ntiles) + 7) & ~7u : blocks_for((long)ntiles)) *
                           groups;
  if (nblocks >= 0x80000000ull) return hipErrorInvalidValue;
  hipLaunchKernelGGL((k_bconv<MT, COG, EPI, DUMP>), dim3((unsigned)nblocks), dim3(kBlock), 0, s, a, b0, b1);
  return hipGetLastError();
}

template <int MT, int EPI, bool DUMP>
hipError_t go_bconv_cog(const BconvArgs& a, int cog, hipStream_t s) {
  switch (cog) {
    case 8: return go_bconv<MT, 8, EPI, DUMP>(a, s);
    case 16: return go_bconv<MT, 16, EPI, DUMP>(a, s);
    case 32:
      // a 2x2 block with 32 channels needs more than 256 VGPRs
      if constexpr (MT == 1) return go_bconv<MT, 32, EPI, DUMP>(a, s);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_bconv(const BconvArgs& a, int epi, int mt, int cog, bool dump, hipStream_t s) {
  if (a.N <= 0 || a.H <= 0 || a.W <= 0) return hipSuccess;
  // byte offsets are 32-bit and 0x80000000 marks "reads 0": tensors stay below 2 GiB
  if ((size_t)a.N * a.H * a.W * (a.cw0 > 0 ? a.cw0 : 1) * 4 >= 0x80000000ull) return hipErrorInvalidValue;
  if (a.ntot && (a.n0 < 0 || a.n0 + a.N > a.ntot)) return hipErrorInvalidValue;
  const int nrel = a.ntot ? a.ntot - a.n0 : a.N;
  if (a.in1 && (size_t)(nrel * a.h1 * a.w1 + 1) * a.cw1 * 4 >= 0x80000000ull) return hipErrorInvalidValue;
  if (a.in1 && a.padoff != 0x80000000u && a.padoff != (uint32_t)((size_t)nrel * a.h1 * a.w1 * a.cw1 * 4))
    return hipErrorInvalidValue;
  if (a.pair && a.cw0 != 1) return hipErrorInvalidValue;  // a first segment of one half-filled word
  // a dump launch stores every P (and every pooled P) it computes: no null target
  if ((dump || epi == EPI_P) && !a.P) return hipErrorInvalidValue;
  if (dump && (epi == EPI_POOL || epi == EPI_RXPOOL) && !a.P2) return hipErrorInvalidValue;
  switch (epi) {
    case EPI_FOLD:
      if (mt == 1) return dump ? go_bconv_cog<1, EPI_FOLD, true>(a, cog, s) : go_bconv_cog<1, EPI_FOLD, false>(a, cog, s);
      if (mt == 2) return dump ? go_bconv_cog<2, EPI_FOLD, true>(a, cog, s) : go_bconv_cog<2, EPI_FOLD, false>(a, cog, s);
      break;
    case EPI_POOL:
      if (mt == 2) return dump ? go_bconv_cog<2, EPI_POOL, true>(a, cog, s) : go_bconv_cog<2, EPI_POOL, false>(a, cog, s);
      break;
    case EPI_HEAD:
      if (mt != 1) break;
      if (cog == 16) return dump ? go_bconv<1, 16, EPI_HEAD, true>(a, s) : go_bconv<1, 16, EPI_HEAD, false>(a, s);
      if (cog == 32) return dump ? go_bconv<1, 32, EPI_HEAD, true>(a, s) : go_bconv<1, 32, EPI_HEAD, false>(a, s);
      break;
    case EPI_P:
      if (mt == 1) return go_bconv_cog<1, EPI_P, false>(a, cog, s);
      if (mt == 2) return go_bconv_cog<2, EPI_P, false>(a, cog, s);
      break;
    case EPI_RX:
      if (!a.res || !a.eA) break;
      if (mt == 1) return dump ? go_bconv_cog<1, EPI_RX, true>(a, cog, s) : go_bconv_cog<1, EPI_RX, false>(a, cog, s);
      break;
    case EPI_RXPOOL:
      if (!a.res || !a.eA || !a.dA || !a.dout) break;
      if (mt == 2) return dump ? go_bconv_cog<2, EPI_RXPOOL, true>(a, cog, s)
                               : go_bconv_cog<2, EPI_RXPOOL, false>(a, cog, s);
      break;
    case EPI_RXHEAD:
      if (mt != 1 || !a.res || !a.eA || a.cout > cog) break;
      if (cog == 16) return dump ? go_bconv<1, 16, EPI_RXHEAD, true>(a, s) : go_bconv<1, 16, EPI_RXHEAD, false>(a, s);
      if (cog == 32) return dump ? go_bconv<1, 32, EPI_RXHEAD, true>(a, s) : go_bconv<1, 32, EPI_RXHEAD, false>(a, s);
      break;
  }
  return hipErrorInvalidValue;
}

#ifndef BNN_MWR
#define BNN_MWR 2
#endif
#ifndef BNN_MWC
#define BNN_MWC 2
#endif

// compute units of the current device (cached per device)
int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev]) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cus[dev] = v;
  }
  return cus[dev];
}

hipError_t launch_real(const RealArgs& a, hipStream_t s) {
  if ((long)a.N * a.H * a.W <= 0) return hipSuccess;
  const size_t xbytes = a.pcols > 0 ? (size_t)a.cin * a.sH * a.sW * 4 : (size_t)a.N * a.cin * a.H * a.W * 4;
  if (xbytes >= 0x80000000ull) return hipErrorInvalidValue;  // out-of-range offsets must stay distinct
  // 16-byte staging: every 4-column group of the input lies wholly inside
  // or wholly outside the image when the row width is a multiple of 4
  const int rowlen = a.pcols > 0 ? a.sW : a.W;
  const int nchunk = (a.cin + kRealMfmaCI - 1) / kRealMfmaCI;
  if (a.wm && rowlen % 4 == 0 && (uintptr_t)a.x % 16 == 0 && xbytes < kRealFar && nchunk % 3 == 0) {
    const int tilesH = (a.H + 7) / 8, tilesW = (a.W + 31) / 32;
    const long ntile = (long)a.N * tilesH * tilesW;
    if (ntile >= 0x80000000l) return hipErrorInvalidValue;
    const int groups = (a.cout + 15) / 16;
    // two blocks per CU fit; the channel groups share them.  A split batch's
    // parts each take the whole grid too: when they run side by side the
    // later part's blocks start as the earlier's finish, and when they do
    // not, a smaller grid would leave each part at half occupancy (measured
    // 521 vs 526 us for the batch-1024 forward)
    const long share = std::max(1l, 2l * device_cus() / groups);
    dim3 grid((unsigned)std::min(ntile, share), (unsigned)groups);
    if (a.cin % kRealMfmaCI)
      hipLaunchKernelGGL((k_real_mfma4<true>), grid, dim3(256), 0, s, a, (uint32_t)xbytes, tilesH, tilesW, (int)ntile);
    else
      hipLaunchKernelGGL((k_real_mfma4<false>), grid, dim3(256), 0, s, a, (uint32_t)xbytes, tilesH, tilesW, (int)ntile);
    return hipGetLastError();
  }
  if (a.wm) {
    if (xbytes >= kRealFar) return hipErrorInvalidValue;
    constexpr int WR = BNN_MWR, WC = BNN_MWC;
    const int tilesH = (a.H + 4 * WR - 1) / (4 * WR), tilesW = (a.W + 16 * WC - 1) / (16 * WC);
    dim3 grid((unsigned)((long)a.N * tilesH * tilesW), (unsigned)((a.cout + 15) / 16));
    if (a.cin % kRealMfmaCI)
      hipLaunchKernelGGL((k_real_mfma<WR, WC, true, false>), grid, dim3(64 * WR * WC), 0, s, a, (uint32_t)xbytes,
                         tilesH, tilesW);
    else
      hipLaunchKernelGGL((k_real_mfma<WR, WC, false, false>), grid, dim3(64 * WR * WC), 0, s, a, (uint32_t)xbytes,
                         tilesH, tilesW);
    return hipGetLastError();
  }
  const int tilesH = (a.H + RT - 1) / RT, tilesW = (a.W + RW - 1) / RW;
  const int groups = (a.cout + RCO - 1) / RCO;
  constexpr int maxg = 1024 / RLANES;
  const int rg = groups >= maxg ? maxg : groups;
  // blocks split along channels must each cover whole 32-bit output words
  if (groups > rg && (rg * RCO) % 32 != 0) return hipErrorInvalidValue;
  dim3 grid((unsigned)((long)a.N * tilesH * tilesW), (unsigned)((groups + rg - 1) / rg));
  switch (rg) {
#define BNN_RG(k) \
  case k: if constexpr (k <= maxg) hipLaunchKernelGGL(k_real_conv<k>, grid, dim3(RLANES * k), 0, s, a, (uint32_t)xbytes, tilesH, tilesW); break;
    BNN_RG(1) BNN_RG(2) BNN_RG(3) BNN_RG(4) BNN_RG(5) BNN_RG(6) BNN_RG(7) BNN_RG(8)
#undef BNN_RG
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_proj(const ProjArgs& a, hipStream_t s) {
  const long nq = (long)a.N * a.H * a.W;
  if (nq <= 0 || a.cout <= 0) return hipSuccess;
  if (!a.x0 || !a.w || !a.out || a.c0 < 0 || a.c0 > a.cin || (a.c0 < a.cin && !a.x1)) return hipErrorInvalidValue;
  // 32-bit buffer offsets, 0x80000000 past every source ("reads 0")
  if (a.ntot && (a.n0 < 0 || a.n0 + a.N > a.ntot)) return hipErrorInvalidValue;
  const long ntot = a.ntot ? a.ntot : a.N;
  if ((long)a.c0 * ntot * a.H * a.W * 4 >= 0x80000000l ||
      (a.x1 && (long)(a.cin - a.c0) * ntot * a.h1 * a.w1 * 4 >= 0x80000000l))
    return hipErrorInvalidValue;
  if ((long)((a.cout + 15) / 16) * ((a.cin + 3) / 4) * 256 >= 0x80000000l) return hipErrorInvalidValue;
  const int ngrp = (a.cout + 15) / 16;
  const long waves = (nq + 63) / 64;
  // groups per wave: all of them while the launch still has ~2048 waves
  // (each output is a chain of cin dependent steps, so deep layers with few
  // positions need the groups spread over waves)
  int G = 8;
  while (G > 1 && (G / 2 >= ngrp || waves * ((ngrp + G - 1) / G) < 2048)) G /= 2;
  dim3 grid((unsigned)((waves + 3) / 4), (unsigned)((ngrp + G - 1) / G));
  switch (G) {
    case 1: hipLaunchKernelGGL(k_proj<1>, grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL(k_proj<2>, grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL(k_proj<4>, grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL(k_proj<8>, grid, dim3(256), 0, s, a); break;
  }
  return hipGetLastError();
}

hipError_t launch_react_epi(const void* acc, int kind, const float* res, float* out, int C, long HW,
                            const float* A, const float* B, const float* move1, const float* prelu_w, int form,
                            hipStream_t s) {
  const long n = (long)C * HW;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_react_epi, dim3(blocks_for(n)), dim3(kBlock), 0, s, acc, kind, res, out, C, HW, A, B, move1,
                     prelu_w, form);
  return hipGetLastError();
}

hipError_t launch_react_tap(const float* x, int8_t* out, int C, long HW, const float* rsign, hipStream_t s) {
  const long n = (long)C * HW;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_react_tap, dim3(blocks_for(n)), dim3(kBlock), 0, s, x, out, C, HW, rsign);
  return hipGetLastError();
}

hipError_t launch_maxpool_real(const float* x, float* out, int C, int H, int W, int k, int stride, hipStream_t s) {
  if (k <= 0 || stride <= 0 || H < k || W < k) return hipSuccess;
  const long n = (long)C * ((H - k) / stride + 1) * ((W - k) / stride + 1);
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_maxpool_real, dim3(blocks_for(n)), dim3(kBlock), 0, s, x, out, C, H, W, k, stride);
  return hipGetLastError();
}

hipError_t launch_conv3_chain(const float* x, const int8_t* wsign, const float* alpha, float* out, int cin, int H,
                              int W, int cout, hipStream_t s) {
  const long n = (long)cout * H * W;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_conv3_chain, dim3(blocks_for(n)), dim3(kBlock), 0, s, x, wsign, alpha, out, cin, H, W,
                     cout);
  return hipGetLastError();
}

hipError_t launch_react_in(const RealArgs& a, hipStream_t s) {
  if ((long)a.N * a.H * a.W <= 0) return hipSuccess;
  if (!a.wm || !a.pw || !a.hout) return hipErrorInvalidValue;
  const size_t xbytes = a.pcols > 0 ? (size_t)a.cin * a.sH * a.sW * 4 : (size_t)a.N * a.cin * a.H * a.W * 4;
  if (xbytes >= kRealFar) return hipErrorInvalidValue;
  constexpr int WR = BNN_MWR, WC = BNN_MWC;
  const int tilesH = (a.H + 4 * WR - 1) / (4 * WR), tilesW = (a.W + 16 * WC - 1) / (16 * WC);
  dim3 grid((unsigned)((long)a.N * tilesH * tilesW), (unsigned)((a.cout + 15) / 16));
  if (a.cin % kRealMfmaCI)
    hipLaunchKernelGGL((k_real_mfma<WR, WC, true, true>), grid, dim3(64 * WR * WC), 0, s, a, (uint32_t)xbytes,
                       tilesH, tilesW);
  else
    hipLaunchKernelGGL((k_real_mfma<WR, WC, false, true>), grid, dim3(64 * WR * WC), 0, s, a, (uint32_t)xbytes,
                       tilesH, tilesW);
  return hipGetLastError();
}

// v3 enc1 unit 1, general-order conv already in a.conv: projection chains,
// real epilogue, h planes and the tap bits of unit 2, a thread per pixel.
// The input column of a channel is read once for 16 output channels (their
// chains advance together, each over ci from 0 in order).
__global__ __launch_bounds__(kBlock) void k_react_in_tail(const ReactTailArgs a) {
  const long i = (long)blockIdx.x * kBlock + threadIdx.x;
  const long HW = (long)a.H * a.W;
  if (i >= (long)a.N * HW) return;
  const int n = (int)(i / HW);
  const long p = i - (long)n * HW;
  const int y = (int)(p / a.W), x = (int)(p - (long)y * a.W);
  // the input column: batch [N][cin][H][W], or a patch of the scene cube
  // (rows and columns past the cube read 0)
  const float* xc;
  long cstride;
  bool inside = true;
  if (a.pcols > 0) {
    const int sy = (a.prow0 + n / a.pcols) * a.H + y, sx = (n % a.pcols) * a.W + x;
    inside = sy < a.sH && sx < a.sW;
    xc = a.x + (inside ? (long)sy * a.sW + sx : 0);
    cstride = (long)a.sH * a.sW;
  } else {
    xc = a.x + (long)n * a.cin * HW + p;
    cstride = HW;
  }
  typedef const __attribute__((address_space(4))) float* const_f;
  const const_f pw = (const_f)a.pw;
  const long plane = (long)(a.ntot ? a.ntot : a.N) * HW;
  const int cw = (a.cout + 31) >> 5;
  uint32_t word = 0;
#pragma unroll 1
  for (int c0 = 0; c0 < a.cout; c0 += 16) {
    float acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
#pragma unroll 1
    for (int ci = 0; ci < a.cin; ++ci) {
      const float v = inside ? xc[ci * cstride] : 0.0f;
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[j] = __fmaf_rn(pw[(c0 + j) * a.cin + ci], v, acc[j]);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int co = c0 + j;
      if (co >= a.cout) continue;
      const long at = ((long)n * a.cout + co) * HW + p;
      const float res = acc[j];
      if (a.f32b) a.f32b[at] = res;
      const float t = __fadd_rn(__fmaf_rn(a.A[co], a.conv[at], a.B[co]), res);
      const float h = t >= 0.0f ? t : __fmul_rn(a.slope[co], t);
      a.hout[co * plane + (long)n * HW + p] = h;
      word |= (__fadd_rn(h, a.rsign[co]) > 0.0f ? 1u : 0u) << (co & 31);
      if ((co & 31) == 31 || co == a.cout - 1) {
        a.out[i * cw + (co >> 5)] = word;
        word = 0;
      }
    }
  }
}

hipError_t launch_react_in_tail(const ReactTailArgs& a, hipStream_t s) {
  const long n = (long)a.N * a.H * a.W;
  if (n <= 0) return hipSuccess;
  if (!a.x || !a.pw || !a.conv || !a.A || !a.B || !a.slope || !a.rsign || !a.out || !a.hout || a.cout <= 0 ||
      a.cin <= 0 || (a.ntot && a.ntot < a.N))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_react_in_tail, dim3(blocks_for(n)), dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

int stem_groups_per_wave(int cout) { return std::min(4, (cout + 15) / 16); }

#ifndef BNN_STEM_NQ4
#define BNN_STEM_NQ4 1  // quads in flight at 4 pixels per lane
#endif
#ifndef BNN_STEM_OCC4
#define BNN_STEM_OCC4 4  // waves per SIMD at 4 pixels per lane
#endif
#ifndef BNN_STEM_PX1
#define BNN_STEM_PX1 2  // pixels per lane with one channel group per wave
#endif
#ifndef BNN_STEM_PX2
#define BNN_STEM_PX2 1  // pixels per lane with two channel groups per wave
#endif

template <int G, int PX>
void launch_stem_t(const RealArgs& a, uint32_t xbytes, int ngp, hipStream_t s) {
  constexpr int NQ = PX == 4 ? BNN_STEM_NQ4 : 4;
  constexpr int OCC = G * PX == 1 ? 5 : PX == 4 ? BNN_STEM_OCC4 : 3;
  constexpr int OCCD = OCC < 3 ? OCC : 3;  // the debug variant's float stores need registers
  const long npix = (long)a.N * a.H * a.W;
  const dim3 grid((unsigned)((npix + 256 * PX - 1) / (256 * PX) * (ngp / G)));
  if (a.f32) hipLaunchKernelGGL((k_stem_mfma<G, PX, NQ, OCCD, true>), grid, dim3(256), 0, s, a, xbytes, ngp);
  else hipLaunchKernelGGL((k_stem_mfma<G, PX, NQ, OCC, false>), grid, dim3(256), 0, s, a, xbytes, ngp);
}

hipError_t launch_stem(const RealArgs& a, hipStream_t s) {
  if ((long)a.N * a.H * a.W <= 0) return hipSuccess;
  const size_t xbytes = a.pcols > 0 ? (size_t)a.cin * a.sH * a.sW * 4 : (size_t)a.N * a.cin * a.H * a.W * 4;
  // offsets stay below 2^31 even for the channels read ahead past cin, so
  // a lane outside the image (base offset 2^31) always reads past the buffer
  const size_t cstride = a.pcols > 0 ? (size_t)a.sH * a.sW : (size_t)a.H * a.W;
  if (xbytes + (size_t)(4 * 4 + 4) * 4 * cstride >= 0x80000000ull || !a.wm || a.cin < 1)
    return hipErrorInvalidValue;
  const int G = stem_groups_per_wave(a.cout);
  const int ngp = stem_groups_padded(a.cout);
  // pixels per lane: a lane's pixels must share a patch row and lie inside
  // or outside the input together (patch widths and, for scenes, the scene
  // width are multiples of PX)
  auto fits = [&](int px) { return a.W % px == 0 && (a.pcols == 0 || a.sW % px == 0); };
  int PX = G == 1 ? BNN_STEM_PX1 : G == 2 ? BNN_STEM_PX2 : 1;
  while (PX > 1 && !fits(PX)) PX /= 2;
  const uint32_t xb = (uint32_t)xbytes;
  switch (G * 8 + PX) {
    case 1 * 8 + 4: launch_stem_t<1, 4>(a, xb, ngp, s); break;
    case 1 * 8 + 2: launch_stem_t<1, 2>(a, xb, ngp, s); break;
    case 1 * 8 + 1: launch_stem_t<1, 1>(a, xb, ngp, s); break;
    case 2 * 8 + 2: launch_stem_t<2, 2>(a, xb, ngp, s); break;
    case 2 * 8 + 1: launch_stem_t<2, 1>(a, xb, ngp, s); break;
    case 3 * 8 + 1: launch_stem_t<3, 1>(a, xb, ngp, s); break;
    default: launch_stem_t<4, 1>(a, xb, ngp, s); break;
  }
  return hipGetLastError();
}

hipError_t launch_pack_act(const int8_t* a, uint32_t* out, int N, int C, int H, int W, hipStream_t s) {
  const long n = (long)N * H * W * ((C + 31) >> 5);
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_pack_act, dim3(blocks_for(n)), dim3(kBlock), 0, s, a, out, N, C, H, W);
  return hipGetLastError();
}

hipError_t launch_bconv_generic(const uint32_t* act, const uint32_t* wt, int32_t* P, int cin, int H, int W,
                                int cout, int kh, int kw, int pad, int stride, hipStream_t s) {
  const long Ho = (H + 2 * pad - kh) / stride + 1, Wo = (W + 2 * pad - kw) / stride + 1;
  if (Ho <= 0 || Wo <= 0 || cout <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_bconv_generic, dim3(blocks_for((long)cout * Ho * Wo)), dim3(kBlock), 0, s, act, wt, P,
                     cin, H, W, cout, kh, kw, pad, stride);
  return hipGetLastError();
}

hipError_t launch_bconv_naive(const int8_t* a, const int8_t* w, int32_t* P, int cin, int H, int W, int cout,
                              int kh, int kw, int pad, int stride, hipStream_t s) {
  const long Ho = (H + 2 * pad - kh) / stride + 1, Wo = (W + 2 * pad - kw) / stride + 1;
  if (Ho <= 0 || Wo <= 0 || cout <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_bconv_naive, dim3(blocks_for((long)cout * Ho * Wo)), dim3(kBlock), 0, s, a, w, P, cin,
                     H, W, cout, kh, kw, pad, stride);
  return hipGetLastError();
}

hipError_t launch_real_generic(const float* x, const float* w, const float* alpha, float* out, int cin, int H,
                               int W, int cout, int kh, int kw, int pad, int stride, hipStream_t s) {
  const long Ho = (H + 2 * pad - kh) / stride + 1, Wo = (W + 2 * pad - kw) / stride + 1;
  if (Ho <= 0 || Wo <= 0 || cout <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_real_generic, dim3(blocks_for((long)cout * Ho * Wo)), dim3(kBlock), 0, s, x, w, alpha,
                     out, cin, H, W, cout, kh, kw, pad, stride);
  return hipGetLastError();
}

hipError_t launch_maxpool(const int32_t* P, int32_t* out, int C, int H, int W, int k, int stride,
                          hipStream_t s) {
  const long Ho = (H - k) / stride + 1, Wo = (W - k) / stride + 1;
  if (Ho <= 0 || Wo <= 0 || C <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_maxpool, dim3(blocks_for((long)C * Ho * Wo)), dim3(kBlock), 0, s, P, out, C, H, W, k,
                     stride);
  return hipGetLastError();
}

hipError_t launch_fold_int(const int32_t* P, int8_t* out, int C, int HW, const int32_t* type, const int32_t* t,
                           const int32_t* lo, const int32_t* hi, hipStream_t s) {
  const long n = (long)C * HW;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_fold_int, dim3(blocks_for(n)), dim3(kBlock), 0, s, P, out, C, HW, type, t, lo, hi);
  return hipGetLastError();
}

hipError_t launch_fold_real(const float* x, int8_t* out, int C, int HW, const float* A, const float* B,
                            const float* slope, const float* rsign, hipStream_t s) {
  const long n = (long)C * HW;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_fold_real, dim3(blocks_for(n)), dim3(kBlock), 0, s, x, out, C, HW, A, B, slope, rsign);
  return hipGetLastError();
}

hipError_t launch_head_sep(const HeadArgs& a, hipStream_t s) {
  const long n = (long)a.N * a.H * a.W;
  if (n <= 0) return hipSuccess;
  if (a.bits ? a.cw != (a.cin + 31) / 32 : !a.planes) return hipErrorInvalidValue;
  if (a.bits) hipLaunchKernelGGL(k_head_sep<true>, dim3(blocks_for(n)), dim3(kBlock), 0, s, a);
  else hipLaunchKernelGGL(k_head_sep<false>, dim3(blocks_for(n)), dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_head(const float* a, const float* W, const float* b, float* out, int cin, int HW, int cout,
                       hipStream_t s) {
  const long n = (long)cout * HW;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_head, dim3(blocks_for(n)), dim3(kBlock), 0, s, a, W, b, out, cin, HW, cout);
  return hipGetLastError();
}

}  // namespace bnn
