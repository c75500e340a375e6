// bnn_device.h - device helpers shared by the gfx950 kernel sources.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bnn_kernels.h"

namespace bnn {
namespace {

// gfx9 buffer descriptor word 3 for raw dword access.  A load whose offset
// is at or past `bytes` returns 0 and a store there is dropped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ float ld_f32(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (int)voff, (int)soff, 0));
}
__device__ __forceinline__ uint32_t ld_u32(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs, (int)voff, (int)soff, 0);
}
// n / d for 0 <= n < 2^31 (make_fastdiv)
__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
  return f.d == 1 ? n : (__umulhi(n, f.mul) >> f.shr);
}

// Where the real conv finds patch n: in a batch [N][cin][H][W], or in one
// scene cube [cin][sH][sW] cut into H x W patches (pcols per row), where the
// rows and columns of an edge patch past the cube count as outside (0).
struct InGeom {
  size_t base, cstride;  // element offsets: patch origin, one channel
  int rstride;           // one row
  int ylim, xlim;        // rows / columns of the patch inside the input
};
__device__ __forceinline__ InGeom in_geom(const RealArgs& a, int n) {
  InGeom g;
  if (a.pcols > 0) {
    const int pr = a.prow0 + n / a.pcols, pc = n % a.pcols;
    g.base = (size_t)pr * a.H * a.sW + (size_t)pc * a.W;
    g.cstride = (size_t)a.sH * a.sW;
    g.rstride = a.sW;
    g.ylim = min(a.H, a.sH - pr * a.H);
    g.xlim = min(a.W, a.sW - pc * a.W);
  } else {
    g.base = (size_t)n * a.cin * a.H * a.W;
    g.cstride = (size_t)a.H * a.W;
    g.rstride = a.W;
    g.ylim = a.H;
    g.xlim = a.W;
  }
  return g;
}

}  // namespace
}  // namespace bnn
