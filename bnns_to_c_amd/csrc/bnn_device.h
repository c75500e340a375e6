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

}  // namespace
}  // namespace bnn
