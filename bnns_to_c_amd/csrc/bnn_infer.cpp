// bnn_infer / bnn_infer_stem - command-line drivers, drop-ins for the
// reference's csrc/bnn_infer (csrc/main.c:1-80) and csrc/bnn_infer_stem
// (csrc/main_stem.c:24-88): same arguments, same "rand" input, same stderr
// report.  One source: built with -DBNN_CLI_STEM=1 it is bnn_infer_stem
// (v2 spectral-stem blobs, bnn_model_stem.h).
//
//   bnn_infer weights.blob input.bin|rand output.bin [H W [reps]]
//     input.bin : n_bands*H*W float32, [band,row,col]; "rand" = srand(1234)
//                 uniform [-1,1] (csrc/main.c:39-41)
//     output.bin: n_classes*H*W float32, [class,row,col]
//     reps      : run the forward reps times, report median/min/max
//
// The forward runs on the GPU.  BNN_PROFILE=1 in the environment adds the
// per-kernel table (the reference needs a separate `make profile` build).
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>
#include <algorithm>

#include "bnn_model.h"
#include "bnn_model_stem.h"
#include "bnn_prof.h"

#ifndef BNN_CLI_STEM
#define BNN_CLI_STEM 0
#endif

namespace {
// the one model type this binary drives
template <bool STEM>
struct Api;
template <>
struct Api<false> {
  using M = Model;
  static M* load(const char* p) { return bnn_load(p); }
  static void forward(const M* m, const float* x, int H, int W, float* y) { bnn_forward(m, x, H, W, y); }
  static void release(M* m) { bnn_free(m); }
  static void banner(const M* m, int H, int W, int reps) {
    fprintf(stderr, "# H=%d W=%d bands=%d classes=%d reps=%d\n", H, W, m->n_bands, m->n_classes, reps);
  }
};
template <>
struct Api<true> {
  using M = StemModel;
  static M* load(const char* p) { return bnn_stem_load(p); }
  static void forward(const M* m, const float* x, int H, int W, float* y) { bnn_stem_forward(m, x, H, W, y); }
  static void release(M* m) { bnn_stem_free(m); }
  static void banner(const M* m, int H, int W, int reps) {
    fprintf(stderr, "# [stem] H=%d W=%d bands=%d classes=%d stem_channels=%d reps=%d\n", H, W, m->n_bands,
            m->n_classes, m->stem_conv.Cout, reps);
  }
};
using A = Api<BNN_CLI_STEM != 0>;
}  // namespace

int main(int argc, char** argv) {
  if (argc < 4) {
    fprintf(stderr, "usage: %s weights.blob input.bin|rand output.bin [H W [reps]]\n", argv[0]);
    return 1;
  }
  const int H = argc > 4 ? atoi(argv[4]) : 32;
  const int W = argc > 5 ? atoi(argv[5]) : 32;
  int reps = argc > 6 ? atoi(argv[6]) : 1;
  if (reps < 1) reps = 1;
  const char* pe = getenv("BNN_PROFILE");
  const bool profile = pe && *pe && strcmp(pe, "0") != 0;

  const double t0 = prof_now();
  A::M* m = A::load(argv[1]);
  const double t_load = prof_now() - t0;

  const long n_in = (long)m->n_bands * H * W;
  std::vector<float> input(n_in);
  if (strcmp(argv[2], "rand") == 0) {
    srand(1234);
    for (long i = 0; i < n_in; ++i) input[i] = (float)rand() / (float)RAND_MAX * 2.0f - 1.0f;  // as csrc/main.c: RAND_MAX taken as float
  } else {
    FILE* fi = fopen(argv[2], "rb");
    if (!fi || fread(input.data(), sizeof(float), n_in, fi) != (size_t)n_in) {
      fprintf(stderr, "bad input file\n");
      return 1;
    }
    fclose(fi);
  }

  const long n_out = (long)m->n_classes * H * W;
  std::vector<float> logits(n_out);
  std::vector<double> ts(reps);
  for (int r = 0; r < reps; ++r) {
    if (profile) bnn_prof_enable(r == reps - 1);  // per-op rows of the last rep
    const double f0 = prof_now();
    A::forward(m, input.data(), H, W, logits.data());
    ts[r] = (prof_now() - f0) * 1e3;
  }
  std::sort(ts.begin(), ts.end());
  const double med = ts[reps / 2], tmin = ts[0], tmax = ts[reps - 1];

  const double w0 = prof_now();
  FILE* fo = fopen(argv[3], "wb");
  if (!fo) {
    fprintf(stderr, "cannot open %s\n", argv[3]);
    return 1;
  }
  fwrite(logits.data(), sizeof(float), n_out, fo);
  fclose(fo);
  const double t_write = (prof_now() - w0) * 1e3;

  A::banner(m, H, W, reps);
  fprintf(stderr, "# blob load : %9.3f ms\n", t_load * 1e3);
  fprintf(stderr, "# forward   : %9.3f ms  (median; min %.3f, max %.3f)\n", med, tmin, tmax);
  fprintf(stderr, "# out write : %9.3f ms\n", t_write);
  prof_report(stderr);
  A::release(m);
  return 0;
}
