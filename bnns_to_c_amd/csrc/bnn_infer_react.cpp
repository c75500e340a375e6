// bnn_infer_react - command-line driver for v3 (ReActNet) blobs, a drop-in
// for the reference's csrc/bnn_infer_react (csrc/main_react.c:1-113): same
// arguments, same input specs, same "rand" cube, same stdout report.
//
//   bnn_infer_react <blob> <input> <output.bin> H W [reps]
//     input : [patch<P>:][mem:]FILE or [patch<P>:]rand
//             FILE    float32 [n_bands,H,W] (read whole: the GPU holds the cube)
//             rand    deterministic N(0,1)-like cube, xorshift64 + Box-Muller
//                     (csrc/main_react.c:28-40)
//             patch<P>: independent P x P patches, P a multiple of 16
//     output: float32 logits [n_classes,H,W]
//     reps  : the same image run reps times, median/min/max reported
//
// The forward runs on the GPU.  BNN_PROFILE=1 in the environment adds the
// per-kernel table on stderr.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "bnn_model.h"
#include "bnn_model_react.h"
#include "bnn_prof.h"

namespace {
// the reference's synthetic cube, the same sequence of doubles (libm sqrt,
// log, cos) rounded to float
void fill_rand(float* x, size_t n) {
  uint64_t s = 88172645463325252ull;
  for (size_t i = 0; i < n; ++i) {
    double u[2];
    for (int k = 0; k < 2; ++k) {
      s ^= s << 13;
      s ^= s >> 7;
      s ^= s << 17;
      u[k] = ((s >> 11) + 0.5) / 9007199254740992.0;
    }
    x[i] = (float)(std::sqrt(-2.0 * std::log(u[0])) * std::cos(6.283185307179586 * u[1]));
  }
}
}  // namespace

int main(int argc, char** argv) {
  if (argc < 6) {
    fprintf(stderr, "usage: %s blob input|rand output H W [reps]\n", argv[0]);
    return 2;
  }
  const char *blob = argv[1], *inp = argv[2], *outp = argv[3];
  const int H = atoi(argv[4]), W = atoi(argv[5]);
  const int reps = argc > 6 ? atoi(argv[6]) : 1;
  if (H <= 0 || W <= 0 || reps <= 0) {
    fprintf(stderr, "bad H/W/reps\n");
    return 2;
  }
  const char* pe = getenv("BNN_PROFILE");
  const bool profile = pe && *pe && strcmp(pe, "0") != 0;

  const double t0 = prof_now();
  ModelR* m = bnn_load_react(blob);
  const double t_load = (prof_now() - t0) * 1e3;

  int patchP = 0;
  if (!strncmp(inp, "patch", 5)) {
    patchP = atoi(inp + 5);
    const char* q = strchr(inp, ':');
    if (patchP <= 0 || !q) {
      fprintf(stderr, "bad patch spec '%s' (use patch32:FILE)\n", inp);
      return 2;
    }
    if (patchP % 16) {
      fprintf(stderr, "patch size must be a multiple of 16\n");
      return 2;
    }
    inp = q + 1;
  }
  const bool is_rand = !strcmp(inp, "rand");
  const bool force_mem = !strncmp(inp, "mem:", 4);
  const char* path = force_mem ? inp + 4 : inp;

  const size_t nin = (size_t)m->n_bands * H * W, nout = (size_t)m->n_classes * H * W;
  std::vector<float> in(nin), out(nout);
  if (is_rand) {
    fill_rand(in.data(), nin);
  } else {
    FILE* f = fopen(path, "rb");
    if (!f || fread(in.data(), sizeof(float), nin, f) != nin) {
      fprintf(stderr, "bad input %s\n", path);
      return 1;
    }
    fclose(f);
  }
  std::vector<double> ts(reps);
  for (int r = 0; r < reps; ++r) {
    if (profile) bnn_prof_enable(r == reps - 1);
    const double a = prof_now();
    if (patchP) bnn_forward_react_patched(m, in.data(), H, W, out.data(), patchP);
    else bnn_forward_react(m, in.data(), H, W, out.data());
    ts[r] = (prof_now() - a) * 1e3;
  }
  std::sort(ts.begin(), ts.end());

  FILE* g = fopen(outp, "wb");
  if (!g) {
    fprintf(stderr, "cannot open %s\n", outp);
    return 1;
  }
  fwrite(out.data(), sizeof(float), nout, g);
  fclose(g);

  printf("# load %.1f ms\n", t_load);
  if (patchP) printf("# mode: patch-wise P=%d\n", patchP);
  printf("# forward %dx%d reps=%d  median %.1f ms  min %.1f  max %.1f\n", H, W, reps, ts[reps / 2], ts[0],
         ts[reps - 1]);
  prof_report(stderr);
  bnn_free_react(m);
  return 0;
}
