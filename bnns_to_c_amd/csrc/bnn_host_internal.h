// bnn_host_internal.h - host helpers shared by the v1/v2 engine
// (bnn_host.cpp) and the v3 engine (bnn_react_host.cpp).  Internal: not
// part of the C ABI.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

namespace bnn {

// record an error text for bnn_last_error() and return code
int set_err(int code, const char* fmt, ...);
// print the recorded error and exit(1) (the reference entry points' behaviour)
[[noreturn]] void die();
// true while bnn_prof_enable(1) is in effect
bool prof_enabled();

#define HIP_TRY(expr)                                                                  \
  do {                                                                                 \
    hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess)                                                              \
      return ::bnn::set_err(BNN_EHIP, "%s: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, \
                            __LINE__);                                                 \
  } while (0)

inline int words(int c) { return (c + 31) >> 5; }
inline int pad32(int c) { return (c + 31) & ~31; }

// kidx sign bits (bit k = ci*taps + t) -> [cw0+cw1][pad32(cout)][taps] uint32
// with channel ci at word ci>>5 of the first segment (ci < cs, or all when
// cs == 0) or at word cw0 + ((ci-cs)>>5) of the second (the upsampled half
// of a concat)
std::vector<uint32_t> repack_bin(const uint64_t* kbits, int cin, int cout, int taps, int cs);
// A repack_bin table whose first segment is one word of at most 16
// channels, recast for the popcount kernel's paired taps: that segment
// becomes 5 words per channel, word q holding tap 2q in its low half and tap
// 2q+1 in its high half (tap 8 alone); a concat's second segment follows
// unchanged.
std::vector<uint32_t> pair_taps(const std::vector<uint32_t>& wt, int cout);

}  // namespace bnn
