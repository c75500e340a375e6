// bnn_cli.cpp - the command-line drivers of libbnn_hip.so, one source built
// once per blob family:
//   -DBNN_CLI_FAMILY=1  bnn_infer        v1 blobs  (csrc/main.c)
//   -DBNN_CLI_FAMILY=2  bnn_infer_stem   v2 blobs  (csrc/main_stem.c)
//   -DBNN_CLI_FAMILY=3  bnn_infer_react  v3 blobs  (csrc/main_react.c)
//
// Scripts written against the reference CLIs keep working: the argument
// grammar, exit codes, messages, report lines, output bytes and the two
// synthetic "rand" inputs are the reference's.
//
//   bnn_infer[_stem] BLOB INPUT OUTPUT [H W [REPS]]          (H = W = 32, REPS = 1)
//     INPUT  float32 [n_bands,H,W] file, or "rand"
//   bnn_infer_react  BLOB INPUT OUTPUT H W [REPS]
//     INPUT  [patch<P>:][mem:]FILE or [patch<P>:]rand
//            FILE      streamed into device memory in row strips, so host
//                      memory never holds the cube; mem:FILE reads it whole
//            patch<P>  independent P x P patches, P a positive multiple of 16
//   OUTPUT float32 logits [n_classes,H,W]; the same image runs REPS times and
//   the median, minimum and maximum forward times are reported.
//
// BNN_PROFILE=1 in the environment adds the per-kernel table of the last rep
// (the reference needs a separate profiling build for it).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <ctime>
#include <vector>

#include "bnn_model.h"
#include "bnn_model_react.h"
#include "bnn_model_stem.h"
#include "bnn_prof.h"

#ifndef BNN_CLI_FAMILY
#define BNN_CLI_FAMILY 1
#endif

namespace {

// ------------------------------------------------------------ inputs
// v1/v2 "rand": the C library's rand() after srand(1234), each draw scaled
// to [-1, 1] in float arithmetic: draw / (float)RAND_MAX * 2 - 1
// (csrc/main.c:38-41).  The float division rounds RAND_MAX to 2^31.
void fill_uniform(std::vector<float>& x) {
  const float top = static_cast<float>(RAND_MAX);
  srand(1234);
  for (float& v : x) v = static_cast<float>(rand()) / top * 2.0f - 1.0f;
}

// v3 "rand": a xorshift64 generator (shifts 13, 7, 17 from the fixed seed of
// csrc/main_react.c:28-40) gives two uniforms per value, each its top 53 bits
// placed mid-cell in (0, 1); the cosine branch of the Box-Muller transform
// turns the pair into one N(0, 1) double, rounded to float.
class NormalStream {
 public:
  float next() {
    const double a = uniform();
    const double b = uniform();
    return static_cast<float>(std::sqrt(-2.0 * std::log(a)) * std::cos(kTwoPi * b));
  }

 private:
  double uniform() {
    s_ ^= s_ << 13;
    s_ ^= s_ >> 7;
    s_ ^= s_ << 17;
    return std::ldexp(static_cast<double>(s_ >> 11) + 0.5, -53);
  }
  static constexpr double kTwoPi = 6.283185307179586;
  uint64_t s_ = 88172645463325252ull;
};

void fill_normal(std::vector<float>& x) {
  NormalStream g;
  for (float& v : x) v = g.next();
}

bool read_floats(const char* path, std::vector<float>& x) {
  FILE* f = fopen(path, "rb");
  if (!f) return false;
  const bool ok = fread(x.data(), sizeof(float), x.size(), f) == x.size();
  fclose(f);
  return ok;
}

bool write_floats(const char* path, const std::vector<float>& y) {
  FILE* f = fopen(path, "wb");
  if (!f) return false;
  fwrite(y.data(), sizeof(float), y.size(), f);
  fclose(f);
  return true;
}

// ------------------------------------------------------------ timing
struct Spread {
  double median, lo, hi;
};

// rep times in ms -> the middle one of the sorted list (the upper middle for
// an even count), the smallest and the largest
Spread spread(std::vector<double> ms) {
  std::sort(ms.begin(), ms.end());
  return {ms[ms.size() / 2], ms.front(), ms.back()};
}

bool profiling() {
  const char* e = getenv("BNN_PROFILE");
  return e && *e && strcmp(e, "0") != 0;
}

// runs fwd() reps times and returns each run's wall time in ms; with
// BNN_PROFILE set, the last run records its per-kernel rows
template <class F>
std::vector<double> time_reps(int reps, F&& fwd) {
  const bool prof = profiling();
  std::vector<double> ms;
  ms.reserve(reps);
  for (int r = 0; r < reps; ++r) {
    if (prof) bnn_prof_enable(r + 1 == reps);
    const double t = prof_now();
    fwd();
    ms.push_back((prof_now() - t) * 1e3);
  }
  return ms;
}

// ------------------------------------------------------------ v1 / v2
// bnn_infer and bnn_infer_stem: identical flow over two model types
template <class M>
struct PlainApi;

template <>
struct PlainApi<Model> {
  static constexpr const char* kBlobArg = "weights.blob";
  static Model* load(const char* p) { return bnn_load(p); }
  static void forward(const Model* m, const float* x, int H, int W, float* y) { bnn_forward(m, x, H, W, y); }
  static void release(Model* m) { bnn_free(m); }
  static void banner(const Model* m, int H, int W, int reps) {
    fprintf(stderr, "# H=%d W=%d bands=%d classes=%d reps=%d\n", H, W, m->n_bands, m->n_classes, reps);
  }
};

template <>
struct PlainApi<StemModel> {
  static constexpr const char* kBlobArg = "weights_stem.blob";
  static StemModel* load(const char* p) { return bnn_stem_load(p); }
  static void forward(const StemModel* m, const float* x, int H, int W, float* y) {
    bnn_stem_forward(m, x, H, W, y);
  }
  static void release(StemModel* m) { bnn_stem_free(m); }
  static void banner(const StemModel* m, int H, int W, int reps) {
    fprintf(stderr, "# [stem] H=%d W=%d bands=%d classes=%d stem_channels=%d reps=%d\n", H, W, m->n_bands,
            m->n_classes, m->stem_conv.Cout, reps);
  }
};

// argv: BLOB INPUT OUTPUT [H [W [REPS]]]; missing sizes are 32, reps below 1
// count as 1 (csrc/main.c:23-30)
template <class M>
int run_plain(int argc, char** argv) {
  using Api = PlainApi<M>;
  if (argc < 4) {
    fprintf(stderr, "usage: %s %s input.bin|rand output.bin [H W [reps]]\n", argv[0], Api::kBlobArg);
    return 1;
  }
  const char* const blob_path = argv[1];
  const char* const in_spec = argv[2];
  const char* const out_path = argv[3];
  int dims[3] = {32, 32, 1};
  for (int k = 0; k < 3 && 4 + k < argc; ++k) dims[k] = atoi(argv[4 + k]);
  const int H = dims[0], W = dims[1], reps = std::max(1, dims[2]);

  const double load_t0 = prof_now();
  M* model = Api::load(blob_path);  // exits on a bad blob
  const double load_ms = (prof_now() - load_t0) * 1e3;

  std::vector<float> x((size_t)model->n_bands * H * W);
  if (strcmp(in_spec, "rand") == 0) {
    fill_uniform(x);
  } else if (!read_floats(in_spec, x)) {
    fprintf(stderr, "bad input file\n");
    return 1;
  }
  std::vector<float> y((size_t)model->n_classes * H * W);
  const Spread t = spread(time_reps(reps, [&] { Api::forward(model, x.data(), H, W, y.data()); }));

  const double write_t0 = prof_now();
  if (!write_floats(out_path, y)) {
    fprintf(stderr, "cannot open %s\n", out_path);
    return 1;
  }
  const double write_ms = (prof_now() - write_t0) * 1e3;

  Api::banner(model, H, W, reps);
  fprintf(stderr, "# blob load : %9.3f ms\n", load_ms);
  fprintf(stderr, "# forward   : %9.3f ms  (median; min %.3f, max %.3f)\n", t.median, t.lo, t.hi);
  fprintf(stderr, "# out write : %9.3f ms\n", write_ms);
  prof_report(stderr);
  Api::release(model);
  return 0;
}

// ------------------------------------------------------------ v3
enum class Source { Synthetic, FileWhole, FileStreamed };

struct ReactInput {
  Source source = Source::FileStreamed;
  const char* path = nullptr;
  int patch = 0;  // 0: the whole image at once
};

// "[patch<P>:][mem:]FILE" | "[patch<P>:]rand" (csrc/main_react.c:66-80);
// returns 0 or the exit code after printing the reference's message
int parse_react_input(const char* spec, ReactInput* in) {
  if (strncmp(spec, "patch", 5) == 0) {
    const int P = atoi(spec + 5);
    const char* colon = strchr(spec, ':');
    if (P <= 0 || colon == nullptr) {
      fprintf(stderr, "bad patch spec '%s' (use patch32:FILE)\n", spec);
      return 2;
    }
    if (P % 16 != 0) {
      fprintf(stderr, "patch size must be a multiple of 16\n");
      return 2;
    }
    in->patch = P;
    spec = colon + 1;
  }
  if (strcmp(spec, "rand") == 0) {
    in->source = Source::Synthetic;
  } else if (strncmp(spec, "mem:", 4) == 0) {
    in->source = Source::FileWhole;
    in->path = spec + 4;
  } else {
    in->source = Source::FileStreamed;
    in->path = spec;
  }
  return 0;
}

double monotonic_ms() {
  timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return ts.tv_sec * 1e3 + ts.tv_nsec * 1e-6;
}

// argv: BLOB INPUT OUTPUT H W [REPS]; the report goes to stdout
int run_react(int argc, char** argv) {
  if (argc < 6) {
    fprintf(stderr, "usage: %s blob input|rand output H W [reps]\n", argv[0]);
    return 2;
  }
  const char* const blob_path = argv[1];
  const char* const out_path = argv[3];
  const int H = atoi(argv[4]), W = atoi(argv[5]);
  const int reps = argc > 6 ? atoi(argv[6]) : 1;
  if (H <= 0 || W <= 0 || reps <= 0) {
    fprintf(stderr, "bad H/W/reps\n");
    return 2;
  }

  const double load_t0 = monotonic_ms();
  ModelR* model = bnn_load_react(blob_path);  // exits on a bad blob
  const double load_ms = monotonic_ms() - load_t0;

  ReactInput in;
  if (const int rc = parse_react_input(argv[2], &in)) return rc;
  std::vector<float> y((size_t)model->n_classes * H * W);
  std::vector<double> ms;

  if (in.source == Source::FileStreamed) {
    FILE* f = fopen(in.path, "rb");
    if (!f) {
      fprintf(stderr, "cannot open %s\n", in.path);
      return 1;
    }
    ms = time_reps(reps, [&] {
      if (in.patch) bnn_forward_react_patched_file(model, f, H, W, y.data(), in.patch);
      else bnn_forward_react_file(model, f, H, W, y.data());
    });
    fclose(f);
  } else {
    std::vector<float> x((size_t)model->n_bands * H * W);
    if (in.source == Source::Synthetic) {
      fill_normal(x);
    } else if (!read_floats(in.path, x)) {
      fprintf(stderr, "bad input %s\n", in.path);
      return 1;
    }
    ms = time_reps(reps, [&] {
      if (in.patch) bnn_forward_react_patched(model, x.data(), H, W, y.data(), in.patch);
      else bnn_forward_react(model, x.data(), H, W, y.data());
    });
  }
  const Spread t = spread(ms);

  if (!write_floats(out_path, y)) {
    fprintf(stderr, "cannot open %s\n", out_path);
    return 1;
  }
  printf("# load %.1f ms\n", load_ms);
  if (in.patch) printf("# mode: patch-wise P=%d\n", in.patch);
  printf("# forward %dx%d reps=%d  median %.1f ms  min %.1f  max %.1f\n", H, W, reps, t.median, t.lo, t.hi);
  prof_report(stderr);
  bnn_free_react(model);
  return 0;
}

}  // namespace

static_assert(BNN_CLI_FAMILY >= 1 && BNN_CLI_FAMILY <= 3,
              "BNN_CLI_FAMILY must be 1 (v1), 2 (v2 stem) or 3 (v3 ReActNet)");

int main(int argc, char** argv) {
  switch (BNN_CLI_FAMILY) {
    case 1: return run_plain<Model>(argc, argv);
    case 2: return run_plain<StemModel>(argc, argv);
    default: return run_react(argc, argv);
  }
}
