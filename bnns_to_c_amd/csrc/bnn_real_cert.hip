// bnn_real_cert.hip - the v1 first conv (real input, +-1 weights, 3x3,
// pad 1, real fold) with certified output bits on the fp16 matrix cores.
//
// The reference sums each in-image tap's input channels in order, then the
// taps in row-major order, all in fp32 (csrc/bnn_conv_realin.c:98-111),
// scales by alpha and folds (csrc/bnn_fold.c:62-77); only the fold's bit
// leaves the layer.  This kernel computes an approximation v' of the tap sum
// v together with a bound E >= |v' - v| that holds for every input, and
// asks whether the fold's bit can change between v' - E and v' + E.  The
// host summarises each channel's fold as at most two change points along
// the floats of a range where no step overflows (real_fold_switches: alpha
// * v, A * o + B, the PReLU branch and the final add are each monotone on
// either side of z = 0); an interval in that range holding no change point
// has one bit, the reference's.  Any other output is recomputed in the
// reference's order from the input rows the block still holds in LDS.
//
// v': per input row and wave (32 input channels), x is scaled by 2^(10 - e),
// e the exponent of the largest |x| there, and split into two integer digits
// d1 = rint(u), d0 = rint((u - d1) * 2048), |d1| <= 2048, |d0| <= 1024, each
// exact in fp16.  The f32 16x16x32 f16 MFMA sums digits times +-1 over three
// taps and 32 channels: every partial sum is an integer below 2^18, so the
// matrix core's result is exact whatever its internal order.  The digit sums
// are recombined (2048 Zh + Zl) and scaled back by 2^(e - 21) in fp32.
//
// E = 2^-24 (1 + 2^-8) A + (1 + 2^-8) Q + 2^-109, rounded up, with
//  * A = sum over the output's 3 x 3 x cin window of (cin - ci + 16) |x|,
//    ci the input channel;
//  * Q = half a grid step 2^(e-21) per term: 48 * 2^(e-21) per (input row,
//    wave) of the window;
//  * the reference's roundings: a tap's sum s_k = fl(s_(k-1) + t_k) over
//    channels k = 1 .. cin, started at 0, is off the exact sum by at most
//    sum_(k >= 2) 2^-24 |s_k|, and |s_k| <= (1 + 2^-24)^k sum_(i <= k) |t_i|,
//    so by at most 2^-24 (1 + 2^-16) sum_i (cin - i + 1) |t_i|; the nine
//    tap sums add 8 2^-24 (1 + 2^-16) sum |x| more;
//  * this kernel's: recombination, two row adds, three adds of the
//    four-wave reduction (each at most 2^-24 (sum |x| + Q)); the weight's
//    "+ 16" covers these and the tap adds, 2^-8 the (1 + 2^-16) factors and
//    the roundings of A itself, 2^-110 underflow.
//
// Work split: one block of four waves per (patch, 16-channel group, tile
// of 32 columns); wave w converts a quarter of the input channels.  Rows stream through a ring of
// four LDS row buffers by 16-byte LDS DMA, one row ahead.  Each step
// converts one input row into digits (the shifted operands of the kx = 0 and
// kx = 2 taps come from DPP row shifts, the 16-lane rows being the operand's
// pixel rows), runs 36 MFMAs into per-ky digit sums and adds them into three
// rolling output-row partials.  An output row is complete one step after its
// last input row: each wave writes its partial, its window sum of |x| and
// its Q to LDS (plain stores; float atomics on LDS are several times slower
// here), and after a barrier each wave adds the four in wave order for a
// quarter of the row, folds, certifies and writes the bits.
//
// Rows wider than 32 (HALO): each block takes 32 output columns, its window
// the same 32 columns (128-byte aligned rows of each channel), and the two
// columns either side of it (halo) arrive beside each row, one float per
// channel and side; they are converted like the window's values, and the
// lanes at the window's ends take them, instead of the zero padding, as
// their kx = 0 / kx = 2 operands and window sums.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <type_traits>

#include "bnn_device.h"
#include "bnn_kernels.h"

namespace bnn {
namespace {

typedef _Float16 cert_f16x8 __attribute__((ext_vector_type(8)));
typedef float cert_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t cert_u32x4 __attribute__((ext_vector_type(4)));

constexpr int kCertRing = 4;                  // input rows in LDS
constexpr uint32_t kCertFar = 0x7FFFFFF0u;    // DMA offset that reads zeros

__device__ __forceinline__ cert_f16x8 as_h8(cert_u32x4 v) { return __builtin_bit_cast(cert_f16x8, v); }

template <int CTRL, bool ZERO>
__device__ __forceinline__ uint32_t dpp(uint32_t old, uint32_t src) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)src, CTRL, 0xF, 0xF, ZERO);
}
// a DPP move whose lanes all take a source lane or 0 (bound_ctrl), so no
// old value has to be placed in the destination first
template <int CTRL>
__device__ __forceinline__ uint32_t dmov(uint32_t src) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)src, CTRL, 0xF, 0xF, true);
}
constexpr int kShl1 = 0x101, kShr1 = 0x111, kRor1 = 0x121;
// halo of one ring slot: [channel 128][side 2] floats
constexpr uint32_t kHaloSlot = 128 * 2 * 4;

// Pixel layout of the operands: lane p of a 16-lane row holds pixel 2p of
// the even segment (s = 0) and pixel 2p + 1 of the odd segment (s = 1).
// The left neighbour (kx = 0) of pixel 2p is the odd segment one lane down
// (lane 0: pixel -1, read as 0), of pixel 2p + 1 the even segment's own
// lane; the right neighbour (kx = 2) of pixel 2p is the odd segment's own
// lane, of 2p + 1 the even segment one lane up (lane 15: pixel 32, read as
// 0).  So each direction moves one segment by one lane, and the moved-in
// zeros are exactly the zero padding of a 32-column window.
__device__ __forceinline__ void lane_down(const cert_u32x4& a, cert_u32x4& o) {
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = dmov<kShr1>(a[i]);
}
__device__ __forceinline__ void lane_up(const cert_u32x4& a, cert_u32x4& o) {
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = dmov<kShl1>(a[i]);
}
// the same with a halo: the lane whose neighbour lies outside the window
// (lane 0 moving down, lane 15 moving up, in each 16-lane row) keeps h
__device__ __forceinline__ void lane_down_h(const cert_u32x4& a, const cert_u32x4& h, cert_u32x4& o) {
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = dpp<kShr1, false>(h[i], a[i]);
}
__device__ __forceinline__ void lane_up_h(const cert_u32x4& a, const cert_u32x4& h, cert_u32x4& o) {
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = dpp<kShl1, false>(h[i], a[i]);
}

__device__ __forceinline__ float f32_of(uint32_t b) { return __builtin_bit_cast(float, b); }
__device__ __forceinline__ uint32_t bits_of(float f) { return __builtin_bit_cast(uint32_t, f); }
// the number of set bits of m below this lane
__device__ __forceinline__ int mbcnt64(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// the reference's real fold of tap sum v (csrc/bnn_fold.c:62-77, A * o + B
// fused as the reference build does); z is the value before the PReLU branch
__device__ __forceinline__ bool fold_bit(float v, float al, float A, float B, float sl, float rs, float& z) {
  const float o = __fmul_rn(al, v);
  z = __fmaf_rn(A, o, B);
  const float h = z < 0.0f ? __fmul_rn(sl, z) : z;
  return __fadd_rn(h, rs) > 0.0f;
}

// the LDS byte offset of (channel ci, column x) in a row buffer: 16-byte
// column groups of channels whose bits 0 and 1 differ are swapped in halves
// (group g -> g ^ 4).  An operand read takes four consecutive channels, one
// per 16-lane row: with 64 banks the four land in four different 16-bank
// quarters, and with 32 the two channels of each half-wave in different
// 16-bank halves.
__device__ __forceinline__ uint32_t row_swz(int ci) { return (uint32_t)((ci ^ (ci >> 1)) & 1); }
__device__ __forceinline__ uint32_t row_off(int ci, int x) {
  return (uint32_t)ci * 128u + ((uint32_t)((x >> 2) ^ (row_swz(ci) << 2)) << 4) + (uint32_t)(x & 3) * 4u;
}
__device__ __forceinline__ void block_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// s_waitcnt with lgkmcnt 0 and vmcnt untouched (63), or vmcnt N (< 16) and
// lgkmcnt 0
constexpr int kWaitLgkm0 = 0xF | (7 << 4) | (0 << 8) | (3 << 14);

template <int N>
__device__ __forceinline__ void wait_vm_lgkm() {
  static_assert(N >= 0 && N < 16, "vmcnt field");
  __builtin_amdgcn_s_waitcnt(N | (7 << 4) | (0 << 8));
}
extern __shared__ __attribute__((aligned(16))) float cert_lds[];

// sum over the four 16-lane rows, in every lane (two permlane swaps)
__device__ __forceinline__ float rows_sum(float x) {
  const auto r16 = __builtin_amdgcn_permlane16_swap(bits_of(x), bits_of(x), false, false);
  const float y = __fadd_rn(f32_of(r16[0]), f32_of(r16[1]));
  const auto r32 = __builtin_amdgcn_permlane32_swap(bits_of(y), bits_of(y), false, false);
  return __fadd_rn(f32_of(r32[0]), f32_of(r32[1]));
}
// the largest of the lanes' non-negative floats, as bits (which order as
// unsigned integers): within each 16-lane row by rotation, then the four
// rows through scalar registers
__device__ __forceinline__ uint32_t wave_max_bits(float m) {
  uint32_t mb = bits_of(m);
  mb = max(mb, dpp<0x128, false>(mb, mb));  // row_ror:8
  mb = max(mb, dpp<0x124, false>(mb, mb));  // row_ror:4
  mb = max(mb, dpp<0x122, false>(mb, mb));  // row_ror:2
  mb = max(mb, dpp<kRor1, false>(mb, mb));
  return max(max((uint32_t)__builtin_amdgcn_readlane((int)mb, 0), (uint32_t)__builtin_amdgcn_readlane((int)mb, 16)),
             max((uint32_t)__builtin_amdgcn_readlane((int)mb, 32), (uint32_t)__builtin_amdgcn_readlane((int)mb, 48)));
}
// per-pixel value (pixel 2p + s in v[s]) plus its left and right neighbours
// (HALO: lane 0's left and lane 15's right neighbour is h, the halo's)
template <bool HALO>
__device__ __forceinline__ void window3(const float (&v)[2], float h, float (&o)[2]) {
  const float l = f32_of(HALO ? dpp<kShr1, false>(bits_of(h), bits_of(v[1])) : dmov<kShr1>(bits_of(v[1])));  // pixel 2p - 1
  const float r = f32_of(HALO ? dpp<kShl1, false>(bits_of(h), bits_of(v[0])) : dmov<kShl1>(bits_of(v[0])));  // pixel 2p + 2
  const float c = __fadd_rn(v[0], v[1]);
  o[0] = __fadd_rn(c, l);
  o[1] = __fadd_rn(c, r);
}
// a wave's partial of one output row: MFMA result register i of lane
// (channel c, row group g) of segment s, pixel 8 g + 2 i + s, at
// ((s * 4 + g) * 16 + c) * 4 + i, so a lane's four result rows are one
// 16-byte store
__device__ __forceinline__ int part_idx(int s, int g, int c) { return ((s * 4 + g) * 16 + c) * 4; }

// Wave w converts input channels cpw * w .. cpw * w + cpw - 1 (cpw = cin / 4):
// element j of lane (p, gq) is channel cpw * w + 4 j + gq, column 16 s + p;
// elements past the wave's channels read as 0.  GUARD: such elements may
// occur for j < 7 (cpw < 28); otherwise only element 7 can be one.
//
// G = 2 (17 to 32 output channels): one block makes both 16-channel groups
// of its tile from one conversion of the input (two sets of matrix ops, two
// partial sets in LDS, one whole output word per pixel); its recompute
// reads the sign masks and the halo columns from global memory, which
// leaves LDS room for two blocks per CU.
template <bool GUARD, bool HALO, int G>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void k_real_cert(const RealArgs a, uint32_t xbytes, int nld, uint32_t nitems) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int p = lane & 15, gq = lane >> 4;
  const int H = a.H, W = a.W, cin = a.cin, cpw = cin >> 2;
  // rows up to 32 wide: one block per patch, window column = image column;
  // wider rows (HALO): tiles of 32 columns, the window the tile itself
  // (columns outside the image read 0)
  const int ntile = HALO ? (W + 31) / 32 : 1;
  // XCD-aware order: blocks go to the XCDs in turn (block b to XCD b % 8),
  // and XCD x takes the x-th eighth of the work items (patch, tile, group)
  // in order, so a tile's channel groups, which read the same input window
  // and write the two halves of the same output words, run on one XCD side
  // by side, next to the neighbouring tiles whose rows share cache lines
  // with theirs (the halo columns): their reads and writes meet in that
  // XCD's L2
  // (one block per patch keeps the plain order)
  const int ng = (a.cout + 16 * G - 1) / (16 * G);  // blocks per tile
  // a launch of fewer patches than a round of the device holds splits each
  // patch's rows into S parts, one block each (launch_real_cert)
  const int S = a.rsplit > 1 ? a.rsplit : 1;
  const bool xorder = ng > 1 || ntile > 1 || G > 1 || S > 1;
  const uint32_t item = xorder ? (blockIdx.x & 7u) * (gridDim.x >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  if (item >= nitems) return;
  const uint32_t q = item / (uint32_t)ng;
  const int grp = (int)(item - q * (uint32_t)ng), rp = (int)(q % (uint32_t)S), tt = (int)(q / (uint32_t)S);
  const int n = tt / ntile, tile = tt - n * ntile;
  // output rows [y0, y1) of the patch, from input rows ys = y0 - 1 (or 0)
  // to y1 (or H - 1)
  const int rh = (H + S - 1) / S, y0 = rp * rh, y1 = min(H, y0 + rh), ys = max(0, y0 - 1);
  const int wx0 = HALO ? 32 * tile : 0;  // image column of window column 0
  const int vhi = HALO ? min(32, W - wx0) : W;  // output window columns 0 .. vhi - 1
  const uint32_t rb = (uint32_t)nld * 1024u;  // bytes per row buffer
  float* opart = cert_lds + (size_t)kCertRing * rb / 4;  // [group][wave][512]
  float* absw = opart + G * 4 * 512;                     // [wave][32]
  float* qw = absw + 4 * 32;                             // [wave]
  uint32_t* wsl = reinterpret_cast<uint32_t*>(qw + 4);   // G = 1: [channel][tap][4] sign masks
  // HALO: [slot][channel 128][side 2], at byte hal_off, one slot per ring
  // row (G = 1) or two (G = 2: the conversion's and the next row's)
  constexpr int kHS = G == 1 ? kCertRing : 2;
  const uint32_t hal_off = (uint32_t)kCertRing * rb + (G * 4 * 512 + 4 * 32 + 4 + (G == 1 ? 16 * 36 : 0)) * 4u;
  const float* hal = cert_lds + hal_off / 4;
  // G = 2: the 32 channels' fold parameters, [parameter 9][channel 32]
  // (alpha, A, B, slope, rsign, t1, t2, dc, b0), after the halo slots
  float* fpar = cert_lds + hal_off / 4 + (HALO ? kHS * kHaloSlot / 4 : 0);
  typedef __attribute__((address_space(3))) float* lds_f32;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_f32)cert_lds;

  // this wave's operand tables: Bw[g][t] for group g, tap t
  cert_f16x8 Bw[G][9];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint4* src = reinterpret_cast<const uint4*>(a.cwb) + ((size_t)((grp * G + g) * 4 + wv) * 9) * 64 + lane;
#pragma unroll
    for (int t = 0; t < 9; ++t) {
      const uint4 v = src[t * 64];
      Bw[g][t] = as_h8((cert_u32x4){v.x, v.y, v.z, v.w});
    }
  }

  // G = 1: the group's sign masks (16 channels x 9 taps x 4 words) for the
  // reference-order recompute; the first row barrier orders them
  if constexpr (G == 1)
    for (int i = tid; i < 16 * 36; i += 256) wsl[i] = a.cws[(size_t)grp * 16 * 36 + i];

  // DMA: wave w issues the row's 1 KiB loads k = w, w + 4, ... < nld; lane L
  // of load k fetches 16 bytes: channel 8 k + L / 8, column group (L % 8)
  // swapped as in row_off
  const InGeom ig = in_geom(a, n);
  const uint32_t rstr4 = (uint32_t)ig.rstride * 4u;
  uint32_t doff[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int k = wv + 4 * m;
    const int ci = 8 * k + (lane >> 3);
    const int g4 = (lane & 7) ^ (int)(row_swz(ci) << 2);
    const int cg = wx0 + 4 * g4;  // image column of the 16-byte group
    const bool ok = k < nld && ci < cin && cg >= 0 && cg < ig.xlim;
    doff[m] = ok ? (uint32_t)(ig.base + (size_t)ci * ig.cstride + cg) * 4u : kCertFar;
  }
  // HALO: wave w's one load per row brings channels 32 w .. 32 w + 31, lane
  // L channel 32 w + L / 2 at window column -1 (L even) or 32 (L odd)
  uint32_t hoff = kCertFar;
  if (HALO) {
    const int ci = 32 * wv + (lane >> 1), col = (lane & 1) ? wx0 + 32 : wx0 - 1;
    if (ci < cin && col >= 0 && col < ig.xlim) hoff = (uint32_t)(ig.base + (size_t)ci * ig.cstride + col) * 4u;
  }
  const uint64_t xaddr = (uint64_t)(uintptr_t)a.x;
  auto uni = [](uint32_t v) __attribute__((always_inline)) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); };
  typedef uint32_t dma_u32x4 __attribute__((ext_vector_type(4)));
  const dma_u32x4 xsrc = {uni((uint32_t)xaddr), uni((uint32_t)(xaddr >> 32) & 0xFFFFu), uni(xbytes), 0x00020000u};
  auto issue = [&](int y) __attribute__((always_inline)) {
    const uint32_t slot = lds0 + (uint32_t)(y % kCertRing) * rb;
    const bool inrow = y < ig.ylim;
    const uint32_t ro = (uint32_t)y * rstr4;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int k = wv + 4 * m;
      if (k >= nld) break;
      const uint32_t m0v = uni(slot + (uint32_t)k * 1024u);
      const uint32_t vo = (inrow && doff[m] != kCertFar) ? doff[m] + ro : kCertFar;
      const dma_u32x4 rd = xsrc;
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                   :
                   : "s"(m0v), "v"(vo), "s"(rd)
                   : "memory");
    }
    if (HALO && 32 * wv < cin) {
      const uint32_t m0h = uni(lds0 + hal_off + (uint32_t)(y % kHS) * kHaloSlot + (uint32_t)wv * 256u);
      const uint32_t vo = (inrow && hoff != kCertFar) ? hoff + ro : kCertFar;
      const dma_u32x4 rd = xsrc;
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                   :
                   : "s"(m0h), "v"(vo), "s"(rd)
                   : "memory");
    }
  };

  // conversion reads (pixels 2p and 2p + 1 of element j's channel, one
  // 8-byte read) and the lane's valid elements
  const uint32_t rdoff = row_off(cpw * wv + gq, 2 * p);
  uint32_t jvalid = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) jvalid |= (4 * j + gq < cpw ? 1u : 0u) << j;
  // weight of element j's |x| in the window sum: cin - ci + 16 for its
  // channel ci (the bound's weighted sum; exact small integers)
  float wsum[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) wsum[j] = (float)(cin + 16 - (cpw * wv + 4 * j + gq));

  // finalize: lane -> output channel fc of each group, pixels fpx0 and
  // fpx0 + 1.  The fold's bit along [-dc, dc] as at most two change points
  // (real_fold_switches): bit(v) = b0 ^ (v >= t1) ^ (v >= t2) there, so an
  // interval inside [-dc, dc] holding no change point has one bit; b0 < 0
  // marks a channel whose every output is recomputed.  G = 1 holds the
  // lane's channel's parameters in registers, G = 2 reads them from LDS
  // when it folds (fpar, staged here; the first row barrier orders it).
  const int fc = lane & 15, fq = lane >> 4;
  const int fpx0 = 8 * wv + 2 * fq;
  float r_al = 0.0f, r_A = 0.0f, r_B = 0.0f, r_sl = 0.0f, r_rs = 0.0f, r_t1 = 0.0f, r_t2 = 0.0f, r_dc = 0.0f,
        r_b0 = 0.0f;
  if constexpr (G == 1) {
    const int co = 16 * grp + fc;
    r_al = a.alpha[co]; r_A = a.A[co]; r_B = a.B[co]; r_sl = a.slope[co]; r_rs = a.rsign[co];
    r_t1 = a.ct1[co]; r_t2 = a.ct2[co]; r_dc = a.cdc[co]; r_b0 = a.cb0[co];
  } else if (tid < 32) {
    const int co = 32 * grp + tid;
    const float* src[9] = {a.alpha, a.A, a.B, a.slope, a.rsign, a.ct1, a.ct2, a.cdc, a.cb0};
#pragma unroll
    for (int k = 0; k < 9; ++k) fpar[k * 32 + tid] = src[k][co];
  }
  // parameter k of group g for the lane's own channel
  auto fp_own = [&](int k, int g) __attribute__((always_inline)) -> float {
    if constexpr (G == 1) {
      const float rv[9] = {r_al, r_A, r_B, r_sl, r_rs, r_t1, r_t2, r_dc, r_b0};
      return rv[k];
    } else {
      return fpar[k * 32 + 16 * g + fc];
    }
  };
  // 2^-24 (1 + 2^-9 + 2^-19) times the weighted window sum: the 2^-9 covers
  // the round-to-nearest steps of A and Q, the 2^-19 those of E and the room
  // for rounding v -+ E to nearest (with the |v| 2^-22 term below)
  const float cA = 0x1p-24f * (1.0f + 0x1p-9f + 0x1p-19f);
  const int cwo = (a.cout + 31) >> 5;
  const bool whole_word = G == 2 || ((grp & 1) == 0 && grp == ng - 1);
  // the partials of pixels fpx0 (even segment) and fpx0 + 1 (odd, 256 floats
  // on) in a wave's partial: segment row group wv, register fq
  const int i0 = part_idx(0, wv, fc) + fq;

  issue(ys);

  // rolling state, rotated at the end of every step: at step yi, acc[g][c0]
  // holds the partial of output row yi, [cn] of yi + 1 and [cp] of yi - 1;
  // ab / qr the window sums and Q of input rows yi, yi + 1 and yi - 1 alike
  cert_f32x4 acc[G][3][2];
  float ab[3][2], qr[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g][k][0] = acc[g][k][1] = (cert_f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    ab[k][0] = ab[k][1] = 0.0f;
    qr[k] = 0.0f;
  }

  uint32_t nund = 0;  // outputs this wave recomputed
  for (int yi = ys; yi <= y1; ++yi) {
    constexpr int c0 = 0, cn = 1, cp = 2;  // yi % 3, (yi + 1) % 3, (yi - 1) % 3 after rotation
    const bool has = yi < H;
    // row yi landed, this wave's LDS traffic done, then every wave's
    wait_vm_lgkm<0>();
    block_barrier();
    if (yi + 1 < H && yi + 1 <= y1) issue(yi + 1);

    float abn[2] = {0.0f, 0.0f}, qn = 0.0f;
    if (has) {
      const float* row = cert_lds + (size_t)(yi % kCertRing) * rb / 4;
      float xv[2][8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float2 v = *reinterpret_cast<const float2*>(&row[(rdoff + (uint32_t)j * 512u) / 4]);
        const bool ok = (GUARD || j == 7) ? ((jvalid >> j) & 1u) != 0 : true;
        xv[0][j] = ok ? v.x : 0.0f;
        xv[1][j] = ok ? v.y : 0.0f;
      }
      // HALO: lane 0's left and lane 15's right halo value of element j's
      // channel (0 in the other lanes)
      float hx[8];
      if constexpr (HALO) {
        // every lane reads (the slot holds 128 channels, so every address
        // is inside it), then selects: left to itself the compiler moves
        // each read under its lane condition, eight branches that each wait
        // for their read
        const float* hrow = hal + (size_t)(yi % kHS) * (kHaloSlot / 4);
        float2 hv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) hv[j] = *reinterpret_cast<const float2*>(&hrow[2 * (cpw * wv + 4 * j + gq)]);
#pragma unroll
        for (int j = 0; j < 8; ++j) asm volatile("" : "+v"(hv[j].x), "+v"(hv[j].y));
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const bool ok = ((GUARD || j == 7) ? ((jvalid >> j) & 1u) != 0 : true) && (p == 0 || p == 15);
          hx[j] = ok ? (p == 0 ? hv[j].x : hv[j].y) : 0.0f;
        }
      }
      // the wave's largest |x| (max ignores a NaN, which reaches v' and A as
      // NaN)
      float m = 0.0f, as[2] = {0.0f, 0.0f}, ash = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        m = fmaxf(fmaxf(m, fabsf(xv[0][j])), fabsf(xv[1][j]));
        as[0] = __fmaf_rn(fabsf(xv[0][j]), wsum[j], as[0]);
        as[1] = __fmaf_rn(fabsf(xv[1][j]), wsum[j], as[1]);
        if constexpr (HALO) {
          m = fmaxf(m, fabsf(hx[j]));
          ash = __fmaf_rn(fabsf(hx[j]), wsum[j], ash);
        }
      }
      const uint32_t mw = wave_max_bits(m);
      const bool finite = mw < 0x7F800000u;
      const int e = finite ? max((int)(mw >> 23) - 127, -100) : 127;
      const float sc = f32_of((uint32_t)(127 + 10 - e) << 23);
      const float sb = f32_of((uint32_t)(127 + e - 21) << 23);
      qn = finite ? 48.0f * sb : __builtin_inff();
      // sum |x| over the wave's channels per pixel, then over the three taps
      // of a row
      float ap[2] = {rows_sum(as[0]), rows_sum(as[1])};
      window3<HALO>(ap, HALO ? rows_sum(ash) : 0.0f, abn);

      // digits, packed two per register (HALO: the halo's in hh, hl)
      // (x, y: the high digits' pair, then the low digits')
      auto digits = [&](float x0, float x1) __attribute__((always_inline)) {
        const float u0 = __fmul_rn(x0, sc), u1 = __fmul_rn(x1, sc);
        const float d10 = __builtin_rintf(u0), d11 = __builtin_rintf(u1);
        const float d00 = __builtin_rintf(__fmul_rn(__fsub_rn(u0, d10), 2048.0f));
        const float d01 = __builtin_rintf(__fmul_rn(__fsub_rn(u1, d11), 2048.0f));
        return make_uint2(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(d10, d11)),
                          __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(d00, d01)));
      };
      cert_u32x4 hi[2], lo[2], hh, hl;
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint2 d = digits(xv[s][2 * i], xv[s][2 * i + 1]);
          hi[s][i] = d.x;
          lo[s][i] = d.y;
        }
      if constexpr (HALO) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint2 d = digits(hx[2 * i], hx[2 * i + 1]);
          hh[i] = d.x;
          hl[i] = d.y;
        }
      }
      // digit sums per ky (taps ky * 3 + kx), kx = 1 first, one group at a
      // time
      const cert_f32x4 z4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int g = 0; g < G; ++g) {
      cert_f32x4 zh[3][2], zl[3][2];
#pragma unroll
      for (int ky = 0; ky < 3; ++ky)
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          zh[ky][s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(hi[s]), Bw[g][ky * 3 + 1], z4, 0, 0, 0);
          zl[ky][s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(lo[s]), Bw[g][ky * 3 + 1], z4, 0, 0, 0);
        }
      {
        // kx = 0: even pixels take the odd segment one lane down, odd pixels
        // the even segment
        cert_u32x4 dh, dl;
        if constexpr (HALO) {
          lane_down_h(hi[1], hh, dh);
          lane_down_h(lo[1], hl, dl);
        } else {
          lane_down(hi[1], dh);
          lane_down(lo[1], dl);
        }
#pragma unroll
        for (int ky = 0; ky < 3; ++ky) {
          zh[ky][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(dh), Bw[g][ky * 3], zh[ky][0], 0, 0, 0);
          zl[ky][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(dl), Bw[g][ky * 3], zl[ky][0], 0, 0, 0);
          zh[ky][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(hi[0]), Bw[g][ky * 3], zh[ky][1], 0, 0, 0);
          zl[ky][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(lo[0]), Bw[g][ky * 3], zl[ky][1], 0, 0, 0);
        }
      }
      {
        // kx = 2: even pixels take the odd segment, odd pixels the even
        // segment one lane up
        cert_u32x4 uh, ul;
        if constexpr (HALO) {
          lane_up_h(hi[0], hh, uh);
          lane_up_h(lo[0], hl, ul);
        } else {
          lane_up(hi[0], uh);
          lane_up(lo[0], ul);
        }
#pragma unroll
        for (int ky = 0; ky < 3; ++ky) {
          zh[ky][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(hi[1]), Bw[g][ky * 3 + 2], zh[ky][0], 0, 0, 0);
          zl[ky][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(lo[1]), Bw[g][ky * 3 + 2], zl[ky][0], 0, 0, 0);
          zh[ky][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(uh), Bw[g][ky * 3 + 2], zh[ky][1], 0, 0, 0);
          zl[ky][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(ul), Bw[g][ky * 3 + 2], zl[ky][1], 0, 0, 0);
        }
      }
      // input row yi feeds output rows yi + 1 (ky 0), yi (ky 1), yi - 1 (ky 2)
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          acc[g][cn][s][r] = __fmul_rn(__fmaf_rn(zh[0][s][r], 2048.0f, zl[0][s][r]), sb);
          acc[g][c0][s][r] = __fmaf_rn(__fmaf_rn(zh[1][s][r], 2048.0f, zl[1][s][r]), sb, acc[g][c0][s][r]);
          acc[g][cp][s][r] = __fmaf_rn(__fmaf_rn(zh[2][s][r], 2048.0f, zl[2][s][r]), sb, acc[g][cp][s][r]);
        }
      }
    }
    ab[c0][0] = abn[0];
    ab[c0][1] = abn[1];
    qr[c0] = qn;

    if (yi > y0) {
      // output row r = yi - 1 is complete in acc[g][cp]: each wave leaves its
      // partials, its window sum of |x| (rows yi - 2, yi - 1, yi) and its
      // quantisation bound in LDS
      const int r = yi - 1;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float* mine = opart + (g * 4 + wv) * 512;
#pragma unroll
        for (int s = 0; s < 2; ++s)
          *reinterpret_cast<float4*>(&mine[part_idx(s, gq, p)]) =
              make_float4(acc[g][cp][s][0], acc[g][cp][s][1], acc[g][cp][s][2], acc[g][cp][s][3]);
      }
      if (gq == 0)
        *reinterpret_cast<float2*>(&absw[wv * 32 + 2 * p]) =
            make_float2(__fadd_rn(__fadd_rn(ab[cn][0], ab[cp][0]), ab[c0][0]),
                        __fadd_rn(__fadd_rn(ab[cn][1], ab[cp][1]), ab[c0][1]));
      if (lane == 0) qw[wv] = __fadd_rn(__fadd_rn(qr[cn], qr[cp]), qr[c0]);
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      block_barrier();

      // finalize: the four partials in wave order
      float v[G][2], Aw[2] = {0.0f, 0.0f};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float2 u = *reinterpret_cast<const float2*>(&absw[w * 32 + fpx0]);
        Aw[0] = __fadd_rn(Aw[0], u.x);
        Aw[1] = __fadd_rn(Aw[1], u.y);
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        v[g][0] = v[g][1] = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float t0 = opart[(g * 4 + w) * 512 + i0], t1 = opart[(g * 4 + w) * 512 + i0 + 256];
          v[g][0] = __fadd_rn(v[g][0], t0);
          v[g][1] = __fadd_rn(v[g][1], t1);
        }
      }
      const float4 qq = *reinterpret_cast<const float4*>(qw);
      const float Qs = __fadd_rn(__fadd_rn(qq.x, qq.y), __fadd_rn(qq.z, qq.w));
      // the row's quantisation part of E with its margins, and 2^-109 for
      // underflow
      const float Qc = __fadd_rn(__fmul_rn(Qs, 1.0f + 0x1p-9f + 0x1p-19f), 0x1p-109f);
      uint64_t bm[G][2], um[G][2];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        bool bit[2], unc[2];
        const float t1 = fp_own(5, g), t2 = fp_own(6, g), dc = fp_own(7, g), b0 = fp_own(8, g);
        const bool chan = 16 * (grp * G + g) + fc < a.cout, thr = b0 >= 0.0f, one = b0 > 0.5f;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          // E with room for rounding v -+ E to nearest
          const float Ev = __fmaf_rn(fabsf(v[g][k]), 0x1p-22f, __fmaf_rn(cA, Aw[k], Qc));
          const float lo = __fsub_rn(v[g][k], Ev), hi = __fadd_rn(v[g][k], Ev);
          const bool c1 = lo >= t1, c2 = lo >= t2;
          const bool ok = thr && (hi >= t1) == c1 && (hi >= t2) == c2 && lo >= -dc && hi <= dc;
          bit[k] = (one ^ c1 ^ c2) && chan;
          unc[k] = !ok && chan && fpx0 + k < vhi;
        }
        bm[g][0] = __ballot(bit[0]);
        bm[g][1] = __ballot(bit[1]);
        um[g][0] = __ballot(unc[0]);
        um[g][1] = __ballot(unc[1]);
      }
      uint64_t uany = 0;
#pragma unroll
      for (int g = 0; g < G; ++g) uany |= um[g][0] | um[g][1];
      if (uany) {
        // A is NaN exactly when the window holds a NaN (its terms are |x|
        // times positive weights; such an output is never certified): the
        // reference's sum is then NaN and the fold's bit 0 for any
        // parameters (NaN > 0 is false), so it needs no recompute
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const uint64_t nm = __ballot(Aw[k] != Aw[k]);
#pragma unroll
          for (int g = 0; g < G; ++g) {
            um[g][k] &= ~nm;
            bm[g][k] &= ~nm;
          }
        }
#pragma unroll
        for (int g = 0; g < G; ++g)
          nund += (uint32_t)(__builtin_popcountll(um[g][0]) + __builtin_popcountll(um[g][1]));
      }

      // uncertain outputs: the reference's order, up to seven at a time,
      // lane t < 63 summing tap t % 9 of output t / 9 over the channels from
      // the LDS rows r - 1 .. r + 1 (a row reached by an infinity leaves
      // all its outputs undecided; seven per pass keep 63 of the 64 lanes
      // busy)
      constexpr int kRb = 7;
#pragma unroll
      for (int g = 0; g < G; ++g) {
      while (um[g][0] | um[g][1]) {
        // the batch: the first kRb pending outputs in the order word 0 then
        // word 1 (lane j holds bit j of each), output k's position li + 64
        // which sent to lane k by a forward permute (lanes outside the batch
        // send to lane 63, which no batch reaches)
        // (the lane index is re-derived here, so that none of the batch's
        // lane arithmetic is hoisted into registers held across the row loop)
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const uint64_t u0 = um[g][0], u1 = um[g][1];
        const int p0 = __builtin_popcountll(u0);
        const int nb = min(kRb, p0 + __builtin_popcountll(u1));
        const int r0 = mbcnt64(u0), r1 = p0 + mbcnt64(u1);
        const bool t0 = ((u0 >> ln) & 1u) && r0 < kRb;
        const bool t1 = ((u1 >> ln) & 1u) && r1 < kRb;
        const int v0 = __builtin_amdgcn_ds_permute((t0 ? r0 : 63) << 2, ln);
        const int v1 = __builtin_amdgcn_ds_permute((t1 ? r1 : 63) << 2, ln + 64);
        const uint64_t c0 = __ballot(t0), c1 = __ballot(t1);
        um[g][0] = u0 & ~c0;
        um[g][1] = u1 & ~c1;
        const int ko = ln < p0 ? v0 : v1;  // lane k < nb: output k
        const int kk = ln / 9, tap = ln - 9 * kk;
        const int mo = __builtin_amdgcn_ds_bpermute(kk << 2, ko);
        const int which = mo >> 6, li = mo & 63;
        const int upx = 8 * wv + 2 * (li >> 4) + which;
        float st = 0.0f;
        const int ky = tap / 3, kx = tap - 3 * (tap / 3);
        const int iy = r + ky - 1, ix = upx + kx - 1;
        if (kk < nb && iy >= 0 && iy < H && wx0 + ix >= 0 && wx0 + ix < W) {
          // lane t sums tap t % 9: its four sign-mask words, then the
          // channels in batches of 32 read ahead of their adds (channels
          // 4 m, 4 m + 3 at column offset c0, 4 m + 1, 4 m + 2 at the
          // swapped one, as row_off lays them out).  A last partial batch
          // reads up to 28 channels past cin, inside the block's LDS (a row
          // buffer holds at least cin channels and 11 KiB of partials follow
          // the ring), and adds +0 for them, which leaves a sum that started
          // at +0 unchanged.  HALO: a column outside the window (-1 or 32)
          // reads the row's halo, [channel][side] (G = 1), or global memory
          // (G = 2), instead.
          const uint4 m4 = G == 1 ? *reinterpret_cast<const uint4*>(&wsl[((li & 15) * 9 + tap) * 4])
                                  : *reinterpret_cast<const uint4*>(
                                        &a.cws[(((size_t)(grp * G + g) * 16 + (li & 15)) * 9 + tap) * 4]);
          const bool hcol = HALO && (ix < 0 || ix > 31);
          const int ixr = hcol ? 0 : ix;
          const float* rowp = cert_lds + (size_t)(iy % kCertRing) * rb / 4;
          const float* ch0 = rowp + (row_off(0, ixr) >> 2);       // channels 4 m, 4 m + 3
          const float* ch1 = rowp + (row_off(1, ixr) >> 2) - 32;  // channels 4 m + 1, 4 m + 2
          const float* hp = hal + (size_t)(iy % kHS) * (kHaloSlot / 4) + (ix < 0 ? 0 : 1);
          // (G = 2: the column in global memory by buffer loads, byte offset
          // goff + channel * cs4; outside the input, past the buffer: 0)
          const uint32_t goff = iy < ig.ylim && wx0 + ix < ig.xlim
                                    ? (uint32_t)(ig.base + (size_t)iy * ig.rstride + (wx0 + ix)) * 4u
                                    : kCertFar;
          const uint32_t cs4 = (uint32_t)ig.cstride * 4u;
          for (int cb = 0; cb < cin; cb += 32) {
            float xb[32];
#pragma unroll
            for (int j = 0; j < 32; j += 4) {
              const int c4 = cb + j;
              xb[j] = ch0[c4 * 32];
              xb[j + 1] = ch1[c4 * 32 + 32];
              xb[j + 2] = ch1[c4 * 32 + 64];
              xb[j + 3] = ch0[c4 * 32 + 96];
            }
            if (hcol) {
              if constexpr (G == 1) {
#pragma unroll
                for (int j = 0; j < 32; ++j) xb[j] = hp[2 * (cb + j)];
              } else {
                // (channels past cin are added as +0 below whatever is read)
                const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.x, xbytes);
#pragma unroll
                for (int j = 0; j < 32; ++j) xb[j] = ld_f32(rs, goff + (uint32_t)(cb + j) * cs4, 0u);
              }
            }
            // -x for a clear mask bit: bit j of the inverted word moved to
            // the sign position
            const uint32_t nw = ~(cb < 32 ? m4.x : cb < 64 ? m4.y : cb < 96 ? m4.z : m4.w);
            if (cin - cb >= 32) {
#pragma unroll
              for (int j = 0; j < 32; ++j) st = __fadd_rn(st, f32_of(bits_of(xb[j]) ^ ((nw << (31 - j)) & 0x80000000u)));
            } else {
              const uint32_t live = (1u << (cin - cb)) - 1u;
#pragma unroll
              for (int j = 0; j < 32; ++j) {
                const float xs = f32_of(bits_of(xb[j]) ^ ((nw << (31 - j)) & 0x80000000u));
                st = __fadd_rn(st, ((live >> j) & 1u) ? xs : 0.0f);
              }
            }
          }
        }
        // lane k < nb: output k's taps in order from lanes 9 k .. 9 k + 8,
        // folded with its channel's parameters, the bit then pulled back by
        // the lane of its position
        const int lc = ko & 15;
        float tot = 0.0f;
        const int tb = ln < kRb ? 36 * ln : 0;  // lane 9 k's byte address, k < kRb
#pragma unroll
        for (int t = 0; t < 9; ++t)
          tot = __fadd_rn(tot, f32_of((uint32_t)__builtin_amdgcn_ds_bpermute(tb + 4 * t, (int)bits_of(st))));
        float pv[5];
#pragma unroll
        for (int q = 0; q < 5; ++q) {
          if constexpr (G == 1) {
            const float rv[5] = {r_al, r_A, r_B, r_sl, r_rs};
            pv[q] = f32_of((uint32_t)__builtin_amdgcn_ds_bpermute(lc << 2, (int)bits_of(rv[q])));  // lane c holds channel c
          } else {
            pv[q] = fpar[q * 32 + 16 * g + lc];
          }
        }
        float zz;
        const int ub = ln < nb && fold_bit(tot, pv[0], pv[1], pv[2], pv[3], pv[4], zz) ? 1 : 0;
        // (every lane runs the permutes: a lane outside EXEC reads as 0)
        const int b0 = __builtin_amdgcn_ds_bpermute((r0 & 63) << 2, ub);
        const int b1 = __builtin_amdgcn_ds_bpermute((r1 & 63) << 2, ub);
        const uint64_t s0 = __ballot(t0 && b0);
        const uint64_t s1 = __ballot(t1 && b1);
        bm[g][0] = (bm[g][0] & ~c0) | s0;
        bm[g][1] = (bm[g][1] & ~c1) | s1;
      }
      }

      // lane (channel k, row group fq), k < 2, stores pixel fpx0 + k: its
      // 16 bits of the group (G = 1), or the whole word of both groups
      if (fc < 2 && fpx0 + fc < vhi) {
        const int HW = H * W;
        const size_t pix = (size_t)n * HW + (size_t)r * W + wx0 + fpx0 + fc;
        if constexpr (G == 2) {
          const uint32_t w0 = (uint32_t)((fc ? bm[0][1] : bm[0][0]) >> (16 * fq)) & 0xFFFFu;
          const uint32_t w1 = (uint32_t)((fc ? bm[1][1] : bm[1][0]) >> (16 * fq)) & 0xFFFFu;
          a.out[pix * cwo + grp] = w0 | (w1 << 16);
        } else {
          const uint32_t word = (uint32_t)((fc ? bm[0][1] : bm[0][0]) >> (16 * fq)) & 0xFFFFu;
          uint8_t* dst = reinterpret_cast<uint8_t*>(a.out + pix * cwo) + grp * 2;
          if (whole_word) *reinterpret_cast<uint32_t*>(dst) = word;
          else *reinterpret_cast<uint16_t*>(dst) = (uint16_t)word;
        }
      }
    }
    // next step: output rows yi + 1 and yi, input rows yi - 1 and yi
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        acc[g][cp][s] = acc[g][c0][s];
        acc[g][c0][s] = acc[g][cn][s];
      }
      ab[cn][s] = ab[cp][s];
      ab[cp][s] = ab[c0][s];
    }
    qr[cn] = qr[cp];
    qr[cp] = qr[c0];
  }
  if (a.ucnt && nund && lane == 0) atomicAdd(a.ucnt, (unsigned long long)nund);
}

}  // namespace

namespace {

using CertFn = void (*)(const RealArgs, uint32_t, int, uint32_t);
const CertFn kCertFns[8] = {k_real_cert<false, false, 1>, k_real_cert<true, false, 1>, k_real_cert<false, true, 1>,
                            k_real_cert<true, true, 1>,   k_real_cert<false, false, 2>, k_real_cert<true, false, 2>,
                            k_real_cert<false, true, 2>,  k_real_cert<true, true, 2>};

// A launch's shape: the variant (guard, halo, G = 2 bits), its LDS bytes and
// work items (blocks of a whole patch) per patch.
struct CertShape {
  int var, nld, G;
  size_t lds;
  long per_patch;
};
CertShape cert_shape(int cin, int cout, int W) {
  CertShape c{};
  c.nld = (cin + 7) / 8;
  const bool guard = cin / 4 < 28, halo = W > 32;
  // 17 to 32 output channels: both 16-channel groups in one block
  c.G = cout > 16 && cout <= 32 ? 2 : 1;
  c.lds = (size_t)kCertRing * c.nld * 1024 + (c.G * 4 * 512 + 4 * 32 + 4 + (c.G == 1 ? 16 * 36 : 0)) * 4 +
          (halo ? (c.G == 1 ? kCertRing : 2) * kHaloSlot : 0) + (c.G == 2 ? 9 * 32 * 4 : 0);
  c.var = (guard ? 1 : 0) + (halo ? 2 : 0) + (c.G == 2 ? 4 : 0);
  c.per_patch = (halo ? (W + 31) / 32 : 1) * (long)((cout + 16 * c.G - 1) / (16 * c.G));
  return c;
}

// The kernel asks for more than 64 KiB of LDS: allow it once per variant and
// device (bit d of the variant's mask for device d).
hipError_t cert_attr(int var) {
  static std::atomic<uint64_t> attr[8];
  int dev = 0;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
  const uint64_t bit = 1ull << (dev & 63);
  if (!(attr[var].load(std::memory_order_acquire) & bit)) {
    if (hipError_t e =
            hipFuncSetAttribute((const void*)kCertFns[var], hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        e != hipSuccess)
      return e;
    attr[var].fetch_or(bit, std::memory_order_acq_rel);
  }
  return hipSuccess;
}

// Blocks of the variant resident on the current device at once (its CUs
// times the blocks one CU holds at these LDS bytes), cached per variant and
// row-buffer count (the devices of one process are alike); 0 if unknown.
long cert_slots(const CertShape& c) {
  static std::atomic<long> cache[8][17];
  if (c.nld < 1 || c.nld > 16) return 0;
  long v = cache[c.var][c.nld].load(std::memory_order_acquire);
  if (v) return v;
  int dev = 0, ncu = 0, per_cu = 0;
  if (cert_attr(c.var) != hipSuccess || hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)kCertFns[c.var], 256, c.lds) != hipSuccess)
    return 0;
  v = (long)ncu * per_cu;
  cache[c.var][c.nld].store(v, std::memory_order_release);
  return v;
}

}  // namespace

long real_cert_round(int cin, int cout, int W) {
  const CertShape c = cert_shape(cin, cout, W);
  const long slots = cert_slots(c);
  return slots > 0 ? slots / c.per_patch : 0;
}

hipError_t launch_real_cert(const RealArgs& a, hipStream_t s) {
  if ((long)a.N * a.H * a.W <= 0) return hipSuccess;
  if (!a.cwb || !a.cws || !a.ct1 || !a.ct2 || !a.cb0 || !a.cdc || !a.out || a.f32 || a.hout) return hipErrorInvalidValue;
  const int rowlen = a.pcols > 0 ? a.sW : a.W;
  if (!real_cert_fits(a.cin, a.W, rowlen) || (uintptr_t)a.x % 16) return hipErrorInvalidValue;
  const size_t xbytes = a.pcols > 0 ? (size_t)a.cin * a.sH * a.sW * 4 : (size_t)a.N * a.cin * a.H * a.W * 4;
  if (xbytes >= kCertFar) return hipErrorInvalidValue;
  const CertShape c = cert_shape(a.cin, a.cout, a.W);
  if (hipError_t e = cert_attr(c.var); e != hipSuccess) return e;
  const long npatch_items = (long)a.N * c.per_patch;
  // Row parts: a block's time is its row steps (the kernel is latency-bound,
  // a block alone on its CU takes about as long as two), so a launch that
  // leaves slots of the round empty splits each patch's rows over S = 2 or 4
  // blocks while S times the blocks still fit in one round, each part at
  // least 8 rows (a part re-reads the input row above it: 17 row steps
  // for half of 32 rows against 33 for all of them)
  const long slots = cert_slots(c);
  int S = 1;
  while (S < 4 && slots > 0 && npatch_items * S * 2 <= slots && a.H / (S * 2) >= 8) S *= 2;
  const long nitems = npatch_items * S;
  if (nitems >= 0x7FFFFFF0) return hipErrorInvalidValue;
  RealArgs b = a;
  b.rsplit = S;
  // a multiple of 8 blocks (one per XCD in turn); the padding ones exit
  const bool xorder = c.per_patch > 1 || a.cout > 16 || S > 1;
  const dim3 grid((unsigned)(xorder ? (nitems + 7) / 8 * 8 : nitems));
  hipLaunchKernelGGL(kCertFns[c.var], grid, dim3(256), c.lds, s, b, (uint32_t)xbytes, c.nld, (uint32_t)nitems);
  return hipGetLastError();
}

}  // namespace bnn
