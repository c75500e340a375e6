// Checks real_fold_switches (bnns_to_c_amd/csrc/bnn_kernels.h) against the
// fold it summarises: for random fold parameters, edge-case parameters and
// many probe values v with |v| <= dc, b0 ^ (v >= t1) ^ (v >= t2) must equal
// the fold's bit.  Prints "ok <cases> <probes> fallback <n>" or the first
// mismatch.
#include <cstdio>
#include <random>

#include "bnn_kernels.h"

using namespace bnn;

int main() {
  std::mt19937_64 rng(12345);
  std::uniform_real_distribution<float> U(-1.0f, 1.0f);
  std::uniform_int_distribution<int32_t> O(-0x7F7FFFFF, 0x7F7FFFFF);
  std::uniform_int_distribution<int> E(-40, 40);
  const float specials[] = {0.0f, -0.0f, 1e-45f, -1e-45f, 1e-38f, 1.0f, -1.0f, 3.0e38f, NAN, INFINITY, -INFINITY};
  long probes = 0;
  int cases = 0, failed_models = 0;
  for (int c = 0; c < 20000; ++c) {
    float p[5];
    for (float& x : p) x = U(rng) * std::ldexp(1.0f, E(rng));
    if (c % 7 == 0) p[c / 7 % 5] = specials[(c / 35) % 11];
    if (c % 11 == 0) p[3] = -std::fabs(p[3]);  // negative slope
    if (c % 13 == 0) p[4] = 0.0f;
    const float al = p[0], A = p[1], B = p[2], sl = p[3], rs = p[4];
    float t1, t2, b0, dc;
    real_fold_switches(al, A, B, sl, rs, &t1, &t2, &b0, &dc);
    ++cases;
    if (b0 < 0.0f) { ++failed_models; continue; }
    std::vector<float> vs;
    for (int k = 0; k < 400; ++k) vs.push_back(real_fval(O(rng)));
    for (int k = 0; k < 100; ++k) vs.push_back(dc * U(rng));
    vs.push_back(dc);
    vs.push_back(-dc);
    for (int k = 0; k < 200; ++k) vs.push_back(U(rng) * std::ldexp(1.0f, E(rng)));
    for (float t : {t1, t2})
      if (std::isfinite(t))
        for (int d = -3; d <= 3; ++d) vs.push_back(real_fval(std::min(0x7F7FFFFF, std::max(-0x7F7FFFFF, real_ford(t) + d))));
    for (float s : specials)
      if (std::isfinite(s)) vs.push_back(s);
    for (float v : vs) {
      if (!(std::fabs(v) <= dc)) continue;
      const bool want = real_fold_bit_host(v, al, A, B, sl, rs);
      const bool got = (b0 != 0.0f) ^ (v >= t1) ^ (v >= t2);
      ++probes;
      if (want != got) {
        std::printf("mismatch al=%a A=%a B=%a sl=%a rs=%a v=%a t1=%a t2=%a b0=%g\n", al, A, B, sl, rs, v, t1, t2, b0);
        return 1;
      }
    }
  }
  std::printf("ok %d %ld fallback %d\n", cases, probes, failed_models);
  return 0;
}
