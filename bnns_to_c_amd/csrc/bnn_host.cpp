// bnn_host.cpp - libbnn_hip.so host side: blob parsing (v1 and the v2
// spectral-stem model), device model, the batched forward, the
// debug/profiling paths and the C ABI.
//
// Blob layout and record order: python/bnn2c/blob.py:36-114,159-200 (v1) and
// :204-240 (v2) read the way csrc/bnn_model.c:27-96 and
// csrc/bnn_model_stem.c:79-122 read them (same checks, plus upsampler == 0,
// which the references read but never check, and version == 1 for v1).  The
// forward follows csrc/bnn_model.c:150-253 stage for stage, and for v2
// csrc/bnn_model_stem.c:171-253 (the stem, then enc1.conv1 binary like
// enc2..4); every stage runs as one kernel on the model's HIP stream over a
// batch of N independent patches.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <cstdarg>
#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "bnn_host_internal.h"
#include "bnn_kernels.h"
#include "bnn_model.h"
#include "bnn_model_stem.h"
#include "bnn_prof.h"

using namespace bnn;

// ------------------------------------------------------------------ errors
namespace {
thread_local std::string g_err;
bool g_prof_on = false;
}  // namespace

namespace bnn {
int set_err(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

[[noreturn]] void die() {
  fprintf(stderr, "%s\n", g_err.c_str());
  exit(1);
}

bool prof_enabled() { return g_prof_on; }

std::vector<uint32_t> repack_bin(const uint64_t* kbits, int cin, int cout, int taps, int cs) {
  const int nw = (cin * taps + 63) / 64;
  const int cw0 = words(cs ? cs : cin), cw1 = cs ? words(cin - cs) : 0;
  const int coutp = pad32(cout);
  std::vector<uint32_t> wt((size_t)(cw0 + cw1) * coutp * taps, 0u);
  for (int co = 0; co < cout; ++co)
    for (int ci = 0; ci < cin; ++ci) {
      int w, b;
      if (!cs || ci < cs) { w = ci >> 5; b = ci & 31; }
      else { w = cw0 + ((ci - cs) >> 5); b = (ci - cs) & 31; }
      for (int t = 0; t < taps; ++t) {
        const int k = ci * taps + t;
        if ((kbits[(size_t)co * nw + (k >> 6)] >> (k & 63)) & 1ull)
          wt[((size_t)w * coutp + co) * taps + t] |= 1u << b;
      }
    }
  return wt;
}

std::vector<uint32_t> pair_taps(const std::vector<uint32_t>& wt, int cout) {
  const int coutp = pad32(cout);
  std::vector<uint32_t> wp((size_t)coutp * 5, 0u);
  for (int co = 0; co < coutp; ++co)
    for (int q = 0; q < 5; ++q) {
      uint32_t v = wt[(size_t)co * 9 + 2 * q];
      if (2 * q + 1 < 9) v |= wt[(size_t)co * 9 + 2 * q + 1] << 16;
      wp[(size_t)co * 5 + q] = v;
    }
  wp.insert(wp.end(), wt.begin() + (size_t)coutp * 9, wt.end());
  return wp;
}
}  // namespace bnn

namespace {

// ------------------------------------------------------------ blob reader
struct Reader {
  std::vector<uint8_t> buf;
  size_t off = 0;
  bool bad = false;

  bool fail(const char* what) {
    if (!bad) set_err(BNN_EBLOB, "%s", what);
    bad = true;
    return false;
  }
  bool raw(void* dst, size_t n) {
    if (bad) return false;
    if (n > buf.size() - off) return fail("short read");
    memcpy(dst, buf.data() + off, n);
    off += n;
    return true;
  }
  int i32() {
    int v = 0;
    raw(&v, 4);
    return v;
  }
  // allocate count*elem bytes after checking they are present in the blob
  template <class T>
  T* arr(long long count) {
    if (bad) return nullptr;
    if (count < 0) { fail("negative record dimension"); return nullptr; }
    const long double need = (long double)count * sizeof(T);
    if (need > (long double)(buf.size() - off)) { fail("short read"); return nullptr; }
    T* p = (T*)malloc(count ? (size_t)count * sizeof(T) : 1);
    if (!p) { fail("out of memory"); return nullptr; }
    raw(p, (size_t)count * sizeof(T));
    return p;
  }
};

constexpr int TAG_BIN = 1, TAG_REAL = 2, TAG_ACT = 3, TAG_HEAD = 4;

void read_conv(Reader& r, Conv* c) {
  memset(c, 0, sizeof *c);
  c->tag = r.i32();
  c->Cout = r.i32(); c->Cin = r.i32(); c->kh = r.i32(); c->kw = r.i32();
  c->pad = r.i32(); c->stride = r.i32();
  if (r.bad) return;
  if (c->tag == TAG_BIN) {
    c->nwords = r.i32();
    c->packed = r.arr<uint64_t>((long long)c->Cout * c->nwords);
  } else if (c->tag == TAG_REAL) {
    if (c->Cout < 0 || c->Cin < 0 || c->kh < 0 || c->kw < 0) { r.fail("negative record dimension"); return; }
    c->wsign = r.arr<int8_t>((long long)c->Cout * c->Cin * c->kh * c->kw);
    c->alpha = r.arr<float>(c->Cout);
  } else {
    char m[64];
    snprintf(m, sizeof m, "bad conv tag %d", c->tag);
    r.fail(m);
  }
}

void read_act(Reader& r, Act* a) {
  memset(a, 0, sizeof *a);
  const int tag = r.i32();
  if (!r.bad && tag != TAG_ACT) {
    char m[64];
    snprintf(m, sizeof m, "bad act tag %d", tag);
    r.fail(m);
    return;
  }
  a->kind = r.i32();
  a->C = r.i32();
  if (r.bad) return;
  if (a->C < 0) { r.fail("negative record dimension"); return; }
  if ((long double)a->C * 16 > (long double)(r.buf.size() - r.off)) { r.fail("short read"); return; }
  if (a->kind == 0) {  // any other kind is the real fold (csrc/bnn_model.c:114-124)
    a->type = r.arr<int32_t>(a->C); a->t = r.arr<int32_t>(a->C);
    a->lo = r.arr<int32_t>(a->C); a->hi = r.arr<int32_t>(a->C);
  } else {
    a->A = r.arr<float>(a->C); a->B = r.arr<float>(a->C);
    a->slope = r.arr<float>(a->C); a->rsign = r.arr<float>(a->C);
  }
}

void free_conv(Conv* c) { free(c->packed); free(c->wsign); free(c->alpha); }
void free_act(Act* a) {
  free(a->type); free(a->t); free(a->lo); free(a->hi);
  free(a->A); free(a->B); free(a->slope); free(a->rsign);
}
void free_host(Model* m) {
  for (int i = 0; i < 4; ++i) {
    free_conv(&m->enc_conv1[i]); free_conv(&m->enc_conv2[i]);
    free_act(&m->enc_act1[i]); free_act(&m->enc_act2_skip[i]); free_act(&m->enc_act2_down[i]);
    free_conv(&m->dec_conv1[i]); free_conv(&m->dec_conv2[i]);
    free_act(&m->dec_act1[i]); free_act(&m->dec_act2[i]);
  }
  free_conv(&m->bott_conv1); free_conv(&m->bott_conv2);
  free_act(&m->bott_act1); free_act(&m->bott_act2);
  free(m->head_W); free(m->head_bias);
}

// the v2 records ahead of the body (csrc/bnn_model_stem.c:94-100)
struct StemPart {
  int has_stem = 0, n_stem_layers = 0;
  Conv c{};
  Act a{};
};

// want = 1: a v1 blob into *out; want = 2: a v2 blob, its stem into *st
int parse_blob(const char* path, Model** out, int want = 1, StemPart* st = nullptr) {
  *out = nullptr;
  FILE* f = fopen(path, "rb");
  if (!f) return set_err(BNN_EBLOB, "cannot open %s", path);
  Reader r;
  uint8_t chunk[1 << 16];
  size_t got;
  while ((got = fread(chunk, 1, sizeof chunk, f)) > 0) r.buf.insert(r.buf.end(), chunk, chunk + got);
  fclose(f);
  if (r.buf.size() < 4) return set_err(BNN_EBLOB, "short read");
  if (memcmp(r.buf.data(), "BNNC", 4) != 0) return set_err(BNN_EBLOB, "bad magic");
  r.off = 4;
  Model* m = (Model*)calloc(1, sizeof(Model));
  if (!m) return set_err(BNN_EBLOB, "out of memory");
  m->version = r.i32();
  if (!r.bad && m->version != want) {
    char msg[128];
    if (want == 2)
      snprintf(msg, sizeof msg, "bnn_stem: expected v2 blob, got v%d (use the v1 engine for non-stem models)",
               m->version);
    else if (m->version == 2)
      snprintf(msg, sizeof msg, "unsupported blob version 2 (a spectral-stem model: load it with bnn_stem_load)");
    else
      snprintf(msg, sizeof msg, "unsupported blob version %d", m->version);
    r.fail(msg);
  }
  m->base_channels = r.i32();
  m->n_bands = r.i32(); m->n_classes = r.i32(); m->upsampler = r.i32();
  if (!r.bad && m->upsampler != 0) {
    char msg[64];
    snprintf(msg, sizeof msg, "unsupported upsampler %d (v1 engine runs nearest only)", m->upsampler);
    r.fail(msg);
  }
  if (want == 2) {
    st->has_stem = r.i32(); st->n_stem_layers = r.i32();
    if (!r.bad && (st->has_stem != 1 || st->n_stem_layers != 1))
      r.fail("bnn_stem: only has_stem=1, n_stem_layers=1 supported");
    read_conv(r, &st->c); read_act(r, &st->a);
  }
  for (int i = 0; i < 4; ++i) {
    read_conv(r, &m->enc_conv1[i]); read_act(r, &m->enc_act1[i]);
    read_conv(r, &m->enc_conv2[i]); read_act(r, &m->enc_act2_skip[i]);
    read_act(r, &m->enc_act2_down[i]);
  }
  read_conv(r, &m->bott_conv1); read_act(r, &m->bott_act1);
  read_conv(r, &m->bott_conv2); read_act(r, &m->bott_act2);
  for (int i = 0; i < 4; ++i) {
    read_conv(r, &m->dec_conv1[i]); read_act(r, &m->dec_act1[i]);
    read_conv(r, &m->dec_conv2[i]); read_act(r, &m->dec_act2[i]);
  }
  const int tag = r.i32();
  if (!r.bad && tag != TAG_HEAD) {
    char msg[64];
    snprintf(msg, sizeof msg, "bad head tag %d", tag);
    r.fail(msg);
  }
  m->head_Cout = r.i32(); m->head_Cin = r.i32();
  m->head_W = r.arr<float>((long long)m->head_Cout * m->head_Cin);
  m->head_bias = r.arr<float>(m->head_Cout);
  if (!r.bad && r.off != r.buf.size()) r.fail("trailing bytes in blob");
  if (r.bad) {
    free_host(m);
    free(m);
    if (st) { free_conv(&st->c); free_act(&st->a); }
    return BNN_EBLOB;
  }
  *out = m;
  return BNN_OK;
}

// The chain the forward assumes; the reference trusts the blob instead.
bool conv_ok(const Conv& c, int tag, int cin) {
  return c.tag == tag && c.Cin == cin && c.Cout > 0 && c.kh == 3 && c.kw == 3 && c.pad == 1 &&
         c.stride == 1 && (tag != TAG_BIN || c.nwords == (cin * 9 + 63) / 64);
}
bool act_ok(const Act& a, bool real, int c) { return a.C == c && (real ? a.kind != 0 : a.kind == 0); }

// st: the v2 stem (1x1 real conv from n_bands channels, real fold), after
// which enc1.conv1 is binary
int validate(const Model* m, const StemPart* st = nullptr) {
  if (m->n_bands <= 0 || m->n_classes <= 0) return set_err(BNN_EBLOB, "bad n_bands/n_classes");
  int c = m->n_bands, skipc[4];
  if (st) {
    const Conv& sc = st->c;
    if (sc.tag != TAG_REAL || sc.Cin != c || sc.Cout <= 0 || sc.kh != 1 || sc.kw != 1 || sc.pad != 0 ||
        sc.stride != 1 || !act_ok(st->a, true, sc.Cout))
      return set_err(BNN_EBLOB, "stem does not chain (a 1x1 pad-0 real conv from n_bands, then a real fold)");
    c = sc.Cout;
  }
  for (int i = 0; i < 4; ++i) {
    const Conv &c1 = m->enc_conv1[i], &c2 = m->enc_conv2[i];
    const bool real = i == 0 && !st;
    if (!conv_ok(c1, real ? TAG_REAL : TAG_BIN, c)) return set_err(BNN_EBLOB, "enc%d.conv1 does not chain", i + 1);
    if (!act_ok(m->enc_act1[i], real, c1.Cout)) return set_err(BNN_EBLOB, "enc%d.act1 does not chain", i + 1);
    if (!conv_ok(c2, TAG_BIN, c1.Cout)) return set_err(BNN_EBLOB, "enc%d.conv2 does not chain", i + 1);
    if (!act_ok(m->enc_act2_skip[i], false, c2.Cout) || !act_ok(m->enc_act2_down[i], false, c2.Cout))
      return set_err(BNN_EBLOB, "enc%d.act2 does not chain", i + 1);
    skipc[i] = c = c2.Cout;
  }
  if (!conv_ok(m->bott_conv1, TAG_BIN, c) || !act_ok(m->bott_act1, false, m->bott_conv1.Cout))
    return set_err(BNN_EBLOB, "bottleneck.conv1 does not chain");
  c = m->bott_conv1.Cout;
  if (!conv_ok(m->bott_conv2, TAG_BIN, c) || !act_ok(m->bott_act2, false, m->bott_conv2.Cout))
    return set_err(BNN_EBLOB, "bottleneck.conv2 does not chain");
  c = m->bott_conv2.Cout;
  for (int i = 0; i < 4; ++i) {
    const Conv &c1 = m->dec_conv1[i], &c2 = m->dec_conv2[i];
    if (!conv_ok(c1, TAG_BIN, skipc[3 - i] + c) || !act_ok(m->dec_act1[i], false, c1.Cout))
      return set_err(BNN_EBLOB, "dec%d.conv1 does not chain", 4 - i);
    if (!conv_ok(c2, TAG_BIN, c1.Cout) || !act_ok(m->dec_act2[i], false, c2.Cout))
      return set_err(BNN_EBLOB, "dec%d.conv2 does not chain", 4 - i);
    c = c2.Cout;
  }
  if (m->head_Cin != c || m->head_Cout != m->n_classes) return set_err(BNN_EBLOB, "head does not chain");
  return BNN_OK;
}

// --------------------------------------------------------- host repacking

struct FoldHost {
  std::vector<int32_t> lo;
  std::vector<uint32_t> wid;
};

// bnn_fold_canon's (lo, wid, inv) as one modular interval per channel:
// !((uint32)(P - lo) < wid) == (uint32)(P - (lo + wid)) < 2^32 - wid for every
// P.  An always-true rule (wid 0, inv 1) becomes [2^31, 2^31 + 2^32 - 1),
// which holds every P with |P| < 2^30.  Padded channels keep wid = 0.
FoldHost canon_fold(const Act& a, int coutp) {
  FoldHost f;
  f.lo.assign(coutp, 0);
  f.wid.assign(coutp, 0);
  std::vector<uint8_t> inv(coutp, 0);
  bnn_fold_canon(a.type, a.t, a.lo, a.hi, a.C, f.lo.data(), f.wid.data(), inv.data());
  for (int c = 0; c < a.C; ++c) {
    if (!inv[c]) continue;
    if (f.wid[c] == 0) {
      f.lo[c] = INT32_MIN;
      f.wid[c] = 0xFFFFFFFFu;
    } else {
      f.lo[c] = (int32_t)((uint32_t)f.lo[c] + f.wid[c]);
      f.wid[c] = 0u - f.wid[c];
    }
  }
  return f;
}

// Which binary convs run on the int8 matrix cores (same results as the
// popcount kernel either way): by default a fold or pool conv with
// cout % 64 == 0, an image tile that fits (mfma_conv_fits), rows at least 16
// wide and 64 or more input channels (use_mfma).  BNN_BCONV_MFMA=0 keeps every conv on the popcount
// kernel, =2 takes the matrix cores wherever they fit (both read when a
// model or layer is created).
int mfma_conv_mode() {
  const char* e = getenv("BNN_BCONV_MFMA");
  if (e && !strcmp(e, "0")) return 0;
  if (e && !strcmp(e, "2")) return 2;
  return 1;
}

// a batch splits into parts of at least kSplitMin patches, at most
// kSplitMax of them, on parallel streams (enqueue_forward; measured at batch
// 1024: two parts 4-5% faster than one, four parts of the binary layers 11%
// slower)
constexpr int kSplitMin = 128;
constexpr int kSplitMax = 2;
// the fused middle takes the level-1 layers from this many patches a launch
constexpr int kMidExtMin = 256;

// ------------------------------------------------------------ device model
struct DevBconv {
  int cin = 0, cout = 0, cs = 0, cw0 = 0, cw1 = 0;
  uint32_t* wt = nullptr;
  FoldDev f1{}, f2{};
  MfmaConv mc{};  // int8 matrix-core tables when cout % 64 == 0 (mc.w null otherwise)
  int mfma = 0;   // mfma_conv_mode() at creation
  int pair = 0;   // cin <= 16, no concat: wt holds tap pairs, 5 words per channel
  uint32_t* mw = nullptr;  // the fused middle's table [words][channel group][9][64] (mid layers only)
};

// The fused middle (launch_mid) replaces the ten convs from enc3.c1 to
// dec3.c2 for patches whose level 2 is 8 x 8.  By default it is taken when
// each layer's work fits a block's four waves in one or two passes (at most
// 64 output channels at 8 x 8, 128 at 4 x 4, 256 at 2 x 2: the reference's
// base width 16 and below); BNN_MID=0 keeps the per-layer kernels.
bool mid_mode() {
  const char* e = getenv("BNN_MID");
  return !(e && !strcmp(e, "0"));
}

// With the fused middle, the level-1 layers around it (enc2.c1, enc2.c2,
// dec2.c1, dec2.c2) run inside the same kernel when level 1 is 16 x 16 and
// they have at most 32 output channels (mid_ext_fits); BNN_MIDX=0 keeps
// them as per-layer kernels.
bool midx_mode() {
  const char* e = getenv("BNN_MIDX");
  return !(e && !strcmp(e, "0"));
}

// The certified first conv (launch_real_cert) makes the v1 enc1.conv1 bits
// whenever its shape fits (real_cert_fits); BNN_CERT=0 keeps the exact-order
// matrix-core kernel for them.  The debug forward's float conv output always
// comes from the exact-order kernel.
bool cert_mode() {
  const char* e = getenv("BNN_CERT");
  return !(e && !strcmp(e, "0"));
}

// The int8 matrix-core conv by default where whole forwards measure it
// faster than the popcount kernel: every fold or pool layer that fits with
// rows at least 16 pixels wide and at least two input words (a 64-channel
// K chunk filled).  Config 4 (256 x 256, base 32: thirteen such layers at
// 128, 64, 32 and 16 wide) 2.34 ms against 2.79 with the popcount kernel
// everywhere (dec4.c1 116 against 223 us, dec2.c1 130 against 190); the
// isolated 128 -> 128 pool layer at 32 x 32 (benchmark config 2) 210
// against 288 us.  A 32-channel input fills half a chunk (config 4's
// enc2.c1: 61 against 46 us), and at 8 x 8 (the headline's level 2 when its
// layers run one by one) a tile's staging and epilogue outweigh its one to
// three chunks (enc3.c1 15 against 8 us, forward 0.342 against 0.320 ms).
// BNN_BCONV_MFMA=2 takes it wherever it fits.
bool use_mfma(const DevBconv& L, int epi, int H, int W) {
  return L.mc.w && mfma_conv_fits(L.cout, H, W, epi) && (L.mfma == 2 || (W >= 16 && L.cw0 + L.cw1 >= 2));
}

struct Workspace {
  int N = 0, H = 0, W = 0;
  uint8_t* base = nullptr;
  size_t cap = 0;  // bytes at base
  uint32_t *a1 = nullptr, *skip[4] = {}, *down[4] = {}, *h[4] = {}, *b1 = nullptr, *b2 = nullptr;
  uint32_t *d1[4] = {}, *d2[4] = {};
};

}  // namespace

struct BnnDevice {
  int device = 0;
  hipStream_t stream = nullptr;
  std::vector<void*> allocs;
  // the first stage: v1 enc1.conv1 (3x3) or the v2 stem (1x1), real conv + real fold
  bool stem = false;
  int rcin = 0, rcout = 0;
  uint64_t* rwm = nullptr;  // lane-mask weights (v1: all signs +-1, else null and rw is used)
  float *rw = nullptr, *ralpha = nullptr, *rA = nullptr, *rB = nullptr, *rslope = nullptr, *rrsign = nullptr;
  // the certified first conv's tables (v1, all signs +-1, cin <= 128, cin % 4 == 0), and cert_mode()
  uint16_t* rcwb = nullptr;
  uint32_t* rcws = nullptr;
  float *rct1 = nullptr, *rct2 = nullptr, *rcb0 = nullptr, *rcdc = nullptr;  // its fold summary
  bool cert = false;
  // outputs the certified conv recomputed (device) and certified in all
  // (host), since the last bnn_cert_stats
  unsigned long long* rcnt = nullptr;
  unsigned long long cert_outputs = 0;
  DevBconv e1[4], e2[4], b1, b2, d1[4], d2[4];
  bool mid = false;  // the fused middle applies (mid_fits at load, and mid_mode())
  bool midx = false; // and takes the level-1 layers too (mid_ext_fits, midx_mode())
  float *hw = nullptr, *hb = nullptr;
  int ncls = 0;
  Workspace ws;
  float* stage_in = nullptr;
  size_t stage_in_cap = 0;
  float* stage_out = nullptr;
  size_t stage_out_cap = 0;
  // scene pipeline: pinned host strips, device strip buffers (cube rows in,
  // map rows out), their copy stream and events
  float* pin[2] = {};
  size_t pin_cap = 0;
  float *strip_in[2] = {}, *strip_out[2] = {};
  size_t strip_in_cap[2] = {}, strip_out_cap[2] = {};
  hipStream_t copy = nullptr;
  hipEvent_t ev_copied[2] = {}, ev_free[2] = {}, ev_done[2] = {};
  // the parts of a large batch before the last run their binary layers on
  // these streams, each from the event after its first conv
  hipStream_t side[kSplitMax - 1] = {};
  hipEvent_t ev_conv[kSplitMax - 1] = {}, ev_join[kSplitMax - 1] = {};
  // this device's copy of `scratch` (bnn_forward_device_noalloc), null if
  // its address could not be looked up (scratch_err says why)
  uint8_t* scratch = nullptr;
  std::string scratch_err;
};

struct BnnConvLayer {
  BnnDevice dev;   // owns the allocations
  DevBconv L;
};

namespace {

template <class T>
int dev_upload(BnnDevice* D, T** dst, const T* src, size_t n) {
  void* p = nullptr;
  HIP_TRY(hipMalloc(&p, n ? n * sizeof(T) : 4));
  D->allocs.push_back(p);
  if (n) HIP_TRY(hipMemcpy(p, src, n * sizeof(T), hipMemcpyHostToDevice));
  *dst = (T*)p;
  return BNN_OK;
}

int upload_fold(BnnDevice* D, FoldDev* fd, const Act& a, int coutp) {
  FoldHost f = canon_fold(a, coutp);
  int32_t* lo;
  uint32_t* wid;
  int rc;
  if ((rc = dev_upload(D, &lo, f.lo.data(), f.lo.size()))) return rc;
  if ((rc = dev_upload(D, &wid, f.wid.data(), f.wid.size()))) return rc;
  fd->lo = lo; fd->wid = wid;
  return BNN_OK;
}

int upload_bconv(BnnDevice* D, DevBconv* L, const Conv& c, int cs, const Act* a1, const Act* a2) {
  L->cin = c.Cin; L->cout = c.Cout; L->cs = cs;
  L->cw0 = words(cs ? cs : c.Cin);
  L->cw1 = cs ? words(c.Cin - cs) : 0;
  std::vector<uint32_t> wt = repack_bin(c.packed, c.Cin, c.Cout, 9, cs);
  L->pair = (cs ? cs : c.Cin) <= 16;
  if (L->pair) wt = pair_taps(wt, c.Cout);
  int rc;
  if ((rc = dev_upload(D, &L->wt, wt.data(), wt.size()))) return rc;
  // rules padded to 64 channels (width 0 past cout): the fused middle reads
  // one per lane of a 64-channel group
  const int coutp = (c.Cout + 63) & ~63;
  if (a1 && (rc = upload_fold(D, &L->f1, *a1, coutp))) return rc;
  if (a2 && (rc = upload_fold(D, &L->f2, *a2, coutp))) return rc;
  L->mfma = mfma_conv_mode();
  if (c.Cout % 64 == 0 && L->mfma) {
    std::vector<int8_t> w8(mfma_w_len(c.Cin, c.Cout, cs));
    std::vector<int32_t> st(mfma_s_len(c.Cout));
    mfma_conv_tables(c.packed, c.Cin, c.Cout, cs, w8.data(), st.data());
    int8_t* dw;
    int32_t* ds;
    if ((rc = dev_upload(D, &dw, w8.data(), w8.size()))) return rc;
    if ((rc = dev_upload(D, &ds, st.data(), st.size()))) return rc;
    L->mc = MfmaConv{dw, ds, mfma_npair(L->cw0, L->cw1)};
  }
  return BNN_OK;
}

// the fused middle's weight table: repack_bin's [word][coutp32][tap] as
// [word][channel group of 64][tap][64], zero past cout, so that the 64 lanes
// of a group read consecutive words for one tap and the taps lie at fixed
// distances
int upload_mid_w(BnnDevice* D, DevBconv* L, const Conv& c, int cs) {
  const std::vector<uint32_t> wt = repack_bin(c.packed, c.Cin, c.Cout, 9, cs);
  const int nwd = L->cw0 + L->cw1, cp32 = pad32(c.Cout), ncg = (c.Cout + 63) / 64;
  std::vector<uint32_t> mw((size_t)nwd * ncg * 9 * 64, 0u);
  for (int w = 0; w < nwd; ++w)
    for (int co = 0; co < c.Cout; ++co)
      for (int t = 0; t < 9; ++t)
        mw[(((size_t)w * ncg + co / 64) * 9 + t) * 64 + co % 64] = wt[((size_t)w * cp32 + co) * 9 + t];
  return dev_upload(D, &L->mw, mw.data(), mw.size());
}

// the ten layers of the fused middle, in its order
std::array<DevBconv*, kMidLayers> mid_layers(BnnDevice* D) {
  return {&D->e1[2], &D->e2[2], &D->e1[3], &D->e2[3], &D->b1, &D->b2, &D->d1[0], &D->d2[0], &D->d1[1], &D->d2[1]};
}

// Whether the fused middle takes this model: widths within one or two
// passes of a block's waves per layer, and the concat layers' word split
// matching the tensors the kernel holds (skip words, then upsampled words).
bool mid_fits(BnnDevice* D) {
  const auto L = mid_layers(D);
  // 8 x 8 layers, 4 x 4, 2 x 2, 4 x 4, 8 x 8
  static const int cap[kMidLayers] = {64, 64, 128, 128, 256, 256, 128, 128, 64, 64};
  for (int l = 0; l < kMidLayers; ++l)
    if (L[l]->cout > cap[l]) return false;
  return D->d1[0].cw0 == words(D->e2[3].cout) && D->d1[0].cw1 == words(D->b2.cout) &&
         D->d1[1].cw0 == words(D->e2[2].cout) && D->d1[1].cw1 == words(D->d2[0].cout);
}

// Whether the fused middle can also take the level-1 layers: one group of
// 32 output channels each, paired taps only over a one-word first segment,
// and dec2.c1's concat split as the enc2 skip, then dec3.c2's words.
bool mid_ext_fits(BnnDevice* D) {
  const DevBconv* X[kMidXLayers] = {&D->e1[1], &D->e2[1], &D->d1[2], &D->d2[2]};
  for (int l = 0; l < kMidXLayers; ++l) {
    if (X[l]->cout > 32 || (X[l]->pair && X[l]->cw0 != 1)) return false;
    if ((X[l]->cw1 != 0) != (l == 2)) return false;
  }
  return D->e1[1].cw0 == words(D->e2[0].cout) && D->e2[1].cw0 == words(D->e1[1].cout) &&
         D->d1[2].cw0 == words(D->e2[1].cout) && D->d1[2].cw1 == words(D->d2[1].cout) &&
         D->d2[2].cw0 == words(D->d1[2].cout);
}

// real conv weights.  v2 stem: lane masks of the 1x1 matrix-core kernel
// (signs +1, -1 or 0).  v1 3x3: lane masks for the matrix-core kernel when
// every sign is +-1, else floats in groups of kRealGroup output channels for
// the vector-ALU kernel.  Folds padded to 32.
int upload_real(BnnDevice* D, const Conv& c, const Act& a) {
  D->rcin = c.Cin;
  D->rcout = c.Cout;
  const int tot = (c.Cout + 31) / 32 * 32;
  auto padv = [&](const float* src) {
    std::vector<float> v(tot, 0.0f);
    std::copy(src, src + c.Cout, v.begin());
    return v;
  };
  int rc;
  if (D->stem) {
    std::vector<uint64_t> wm(real_stem_masks_len(c.Cout, c.Cin));
    real_stem_masks(c.wsign, c.Cout, c.Cin, wm.data());
    if ((rc = dev_upload(D, &D->rwm, wm.data(), wm.size()))) return rc;
  } else if (real_conv_signs_only(c.wsign, c.Cout, c.Cin)) {
    std::vector<uint64_t> wm(real_conv_masks_len(c.Cout, c.Cin));
    real_conv_masks(c.wsign, c.Cout, c.Cin, wm.data());
    if ((rc = dev_upload(D, &D->rwm, wm.data(), wm.size()))) return rc;
    if (c.Cin <= 128 && c.Cin % 4 == 0) {
      std::vector<uint16_t> cb(real_cert_b_len(c.Cout));
      std::vector<uint32_t> cs(real_cert_s_len(c.Cout));
      real_cert_tables(c.wsign, c.Cout, c.Cin, cb.data(), cs.data());
      if ((rc = dev_upload(D, &D->rcwb, cb.data(), cb.size()))) return rc;
      if ((rc = dev_upload(D, &D->rcws, cs.data(), cs.size()))) return rc;
    }
  } else {
    std::vector<float> w(real_conv_weights_len(c.Cout, c.Cin));
    real_conv_weights(c.wsign, c.Cout, c.Cin, w.data());
    if ((rc = dev_upload(D, &D->rw, w.data(), w.size()))) return rc;
  }
  std::vector<float> v;
  v = padv(c.alpha); if ((rc = dev_upload(D, &D->ralpha, v.data(), v.size()))) return rc;
  v = padv(a.A); if ((rc = dev_upload(D, &D->rA, v.data(), v.size()))) return rc;
  v = padv(a.B); if ((rc = dev_upload(D, &D->rB, v.data(), v.size()))) return rc;
  v = padv(a.slope); if ((rc = dev_upload(D, &D->rslope, v.data(), v.size()))) return rc;
  v = padv(a.rsign); if ((rc = dev_upload(D, &D->rrsign, v.data(), v.size()))) return rc;
  if (D->rcwb) {
    // the certified kernel's summary of each channel's fold
    const size_t np = (size_t)(c.Cout + 31) / 32 * 32;
    std::vector<float> t1(np, INFINITY), t2(np, INFINITY), b0(np, -1.0f), dc(np, 0.0f);
    for (int co = 0; co < c.Cout; ++co)
      real_fold_switches(c.alpha[co], a.A[co], a.B[co], a.slope[co], a.rsign[co], &t1[co], &t2[co], &b0[co], &dc[co]);
    if ((rc = dev_upload(D, &D->rct1, t1.data(), np))) return rc;
    if ((rc = dev_upload(D, &D->rct2, t2.data(), np))) return rc;
    if ((rc = dev_upload(D, &D->rcb0, b0.data(), np))) return rc;
    if ((rc = dev_upload(D, &D->rcdc, dc.data(), np))) return rc;
    const unsigned long long zero = 0;
    if ((rc = dev_upload(D, &D->rcnt, &zero, 1))) return rc;
  }
  return BNN_OK;
}

void release(BnnDevice* D) {
  if (!D) return;
  if (D->stream) (void)hipStreamSynchronize(D->stream);
  for (hipStream_t q : D->side)
    if (q) (void)hipStreamSynchronize(q);
  for (void* p : D->allocs) (void)hipFree(p);
  D->allocs.clear();
  if (D->ws.base) (void)hipFree(D->ws.base);
  if (D->stage_in) (void)hipFree(D->stage_in);
  if (D->stage_out) (void)hipFree(D->stage_out);
  if (D->copy) (void)hipStreamSynchronize(D->copy);
  for (int k = 0; k < 2; ++k) {
    if (D->pin[k]) (void)hipHostFree(D->pin[k]);
    if (D->strip_in[k]) (void)hipFree(D->strip_in[k]);
    if (D->strip_out[k]) (void)hipFree(D->strip_out[k]);
    if (D->ev_copied[k]) (void)hipEventDestroy(D->ev_copied[k]);
    if (D->ev_free[k]) (void)hipEventDestroy(D->ev_free[k]);
    if (D->ev_done[k]) (void)hipEventDestroy(D->ev_done[k]);
  }
  if (D->copy) (void)hipStreamDestroy(D->copy);
  for (int k = 0; k < kSplitMax - 1; ++k) {
    if (D->ev_conv[k]) (void)hipEventDestroy(D->ev_conv[k]);
    if (D->ev_join[k]) (void)hipEventDestroy(D->ev_join[k]);
    if (D->side[k]) (void)hipStreamDestroy(D->side[k]);
  }
  if (D->stream) (void)hipStreamDestroy(D->stream);
  D->stream = nullptr;
}

// ------------------------------------------------- allocation-free forward
// bnn_forward_device_noalloc keeps its inter-layer tensors in this array, of
// which every GPU holds its own copy from the library's load until the
// process ends.  In host code `scratch` names a host-side stand-in, not
// device memory: each device's address comes from hipGetSymbolAddress, looked
// up once per device (with that device current) when the first model is
// loaded there, and only that address is handed to kernels.
static __device__ __align__(256) uint8_t scratch[BNN_NOALLOC_SCRATCH_BYTES];

std::mutex g_scratch_mu;
std::vector<uint8_t*> g_scratch_dev;  // by device ordinal; null until looked up

int scratch_lookup(int dev, uint8_t** out) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (dev < 0) return set_err(BNN_EHIP, "bad device ordinal %d", dev);
  if ((int)g_scratch_dev.size() <= dev) g_scratch_dev.resize(dev + 1, nullptr);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_err(BNN_EHIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_dev[dev] = (uint8_t*)p;
  }
  *out = g_scratch_dev[dev];
  return BNN_OK;
}

int build_device(Model* m, const StemPart* st = nullptr) {
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
    return set_err(BNN_EHIP, "no HIP device visible: libbnn_hip runs the forward on the GPU only");
  BnnDevice* D = new BnnDevice();
  m->dev = D;
  HIP_TRY(hipGetDevice(&D->device));
  HIP_TRY(hipStreamCreateWithFlags(&D->stream, hipStreamNonBlocking));
  int rc;
  // a failed lookup only disables the allocation-free entry point
  if (scratch_lookup(D->device, &D->scratch)) {
    D->scratch = nullptr;
    D->scratch_err = g_err;
  }
  D->stem = st != nullptr;
  if ((rc = st ? upload_real(D, st->c, st->a) : upload_real(D, m->enc_conv1[0], m->enc_act1[0]))) return rc;
  if ((rc = upload_bconv(D, &D->e2[0], m->enc_conv2[0], 0, &m->enc_act2_skip[0], &m->enc_act2_down[0]))) return rc;
  for (int i = 0; i < 4; ++i) {
    if (i == 0 && !st) continue;  // v1 enc1.conv1 is the real conv above
    if ((rc = upload_bconv(D, &D->e1[i], m->enc_conv1[i], 0, &m->enc_act1[i], nullptr))) return rc;
    if (i && (rc = upload_bconv(D, &D->e2[i], m->enc_conv2[i], 0, &m->enc_act2_skip[i], &m->enc_act2_down[i])))
      return rc;
  }
  if ((rc = upload_bconv(D, &D->b1, m->bott_conv1, 0, &m->bott_act1, nullptr))) return rc;
  if ((rc = upload_bconv(D, &D->b2, m->bott_conv2, 0, &m->bott_act2, nullptr))) return rc;
  for (int i = 0; i < 4; ++i) {
    const int cs = m->enc_conv2[3 - i].Cout;
    if ((rc = upload_bconv(D, &D->d1[i], m->dec_conv1[i], cs, &m->dec_act1[i], nullptr))) return rc;
    if ((rc = upload_bconv(D, &D->d2[i], m->dec_conv2[i], 0, &m->dec_act2[i], nullptr))) return rc;
  }
  D->mid = mid_mode() && mid_fits(D);
  D->midx = D->mid && midx_mode() && mid_ext_fits(D);
  D->cert = cert_mode() && D->rcwb && D->rcws && D->rct1;
  if (D->mid) {
    const auto L = mid_layers(D);
    const Conv* cv[kMidLayers] = {&m->enc_conv1[2], &m->enc_conv2[2], &m->enc_conv1[3], &m->enc_conv2[3],
                                  &m->bott_conv1,   &m->bott_conv2,   &m->dec_conv1[0],  &m->dec_conv2[0],
                                  &m->dec_conv1[1], &m->dec_conv2[1]};
    for (int l = 0; l < kMidLayers; ++l)
      if ((rc = upload_mid_w(D, L[l], *cv[l], L[l]->cs))) return rc;
  }
  D->ncls = m->head_Cout;
  if ((rc = dev_upload(D, &D->hw, m->head_W, (size_t)m->head_Cout * m->head_Cin))) return rc;
  if ((rc = dev_upload(D, &D->hb, m->head_bias, (size_t)m->head_Cout))) return rc;
  HIP_TRY(hipDeviceSynchronize());
  return BNN_OK;
}

// per-level spatial dims: level 0 = input, 1..4 after each pool
void level_dims(int H, int W, int* hs, int* wsz) {
  hs[0] = H; wsz[0] = W;
  for (int l = 1; l <= 4; ++l) { hs[l] = hs[l - 1] / 2; wsz[l] = wsz[l - 1] / 2; }
}

// Lay the inter-layer tensors of an N x H x W forward out from `base` (each
// on a 256-byte boundary) and return the bytes they take; with base null only
// the size is computed.
size_t plan_ws(const Model* m, const BnnDevice* D, Workspace& w, int N, int H, int W, uint8_t* base) {
  int hs[5], ws[5];
  level_dims(H, W, hs, ws);
  size_t off = 0;
  auto add = [&](uint32_t** p, int lvl, int c) {
    if (base) *p = (uint32_t*)(base + off);
    off += ((size_t)N * hs[lvl] * ws[lvl] * words(c) * 4 + 255) & ~(size_t)255;
  };
  add(&w.a1, 0, D->rcout);  // first-stage bits
  for (int i = 0; i < 4; ++i) {
    if (i || D->stem) add(&w.h[i], i, m->enc_conv1[i].Cout);
    add(&w.skip[i], i, m->enc_conv2[i].Cout);
    add(&w.down[i], i + 1, m->enc_conv2[i].Cout);
  }
  add(&w.b1, 4, m->bott_conv1.Cout);
  add(&w.b2, 4, m->bott_conv2.Cout);
  for (int i = 0; i < 4; ++i) {
    add(&w.d1[i], 3 - i, m->dec_conv1[i].Cout);
    add(&w.d2[i], 3 - i, m->dec_conv2[i].Cout);
  }
  if (base) { w.base = base; w.N = N; w.H = H; w.W = W; }
  return off;
}

int ensure_ws(const Model* m, BnnDevice* D, Workspace& w, int N, int H, int W) {
  if (w.base && w.N >= N && w.H == H && w.W == W) return BNN_OK;
  // another shape that fits the allocation is laid out in it anew (work
  // already enqueued on the same stream finishes first; the tiles of one
  // whole image run on one stream)
  const size_t need = plan_ws(m, D, w, N, H, W, nullptr);
  if (w.base && need <= w.cap) {
    uint8_t* base = w.base;
    const size_t cap = w.cap;
    plan_ws(m, D, w, N, H, W, base);
    w.cap = cap;
    return BNN_OK;
  }
  // a forward may still be in flight on a caller's stream
  if (w.base) { HIP_TRY(hipDeviceSynchronize()); (void)hipFree(w.base); w.base = nullptr; w.cap = 0; }
  uint8_t* base = nullptr;
  HIP_TRY(hipMalloc((void**)&base, need));
  plan_ws(m, D, w, N, H, W, base);
  w.cap = need;
  return BNN_OK;
}

// ------------------------------------------------------------ profiling
struct ProfRec {
  std::string label, optype;
  double oe, taps, sec;
};
std::vector<ProfRec> g_prof;

// work-item shape: pool epilogue needs 2x2 blocks, the head one pixel; the
// channel group shrinks until the launch has ~4 waves per SIMD
void pick_shape(int epi, int N, int H, int W, int cout, int* mt, int* cog) {
  *mt = (epi == EPI_POOL) ? 2 : 1;
  if (epi == EPI_HEAD) { *cog = cout <= 16 ? 16 : 32; return; }
  const long tiles = (long)N * ((H + *mt - 1) / *mt) * ((W + *mt - 1) / *mt);
  int c = *mt == 2 ? 16 : 32;
  while (c > 8 && c / 2 >= cout) c /= 2;  // no group wider than the layer
  auto waves = [&](int g) { return ((tiles + 63) / 64) * (long)((cout + g - 1) / g); };
  while (c > 8 && waves(c) < 4096) c /= 2;
  *cog = c;
}

struct Dumps {
  bool on = false;
  float* conv1 = nullptr;
  int32_t* P[32] = {};
  int32_t* P2[4] = {};
};

// Scene mode: the input is one cube [n_bands][sH][sW] cut into patches,
// pcols per row starting at patch row prow0; logits go to the map
// [n_classes][sH][sW]
struct Scene {
  int sH, sW, pcols, prow0;
};

struct Op {
  const char* label;
  const char* optype;
  double oe, taps;
};

// Enqueue the whole forward for N patches on stream s with workspace w.
// Each stage is one kernel; with profiling on, an event pair brackets every
// kernel.
int enqueue_forward(const Model* m, BnnDevice* D, Workspace& w, const float* d_in, int N, int H, int W,
                    float* d_logits, hipStream_t s, Dumps* dmp, std::vector<Op>* ops,
                    std::vector<hipEvent_t>* evs, const Scene* sc = nullptr, int max_parts = kSplitMax) {
  int hs[5], wsz[5];
  level_dims(H, W, hs, wsz);
  auto mark = [&](const char* label, const char* optype, double oe, double taps) -> int {
    if (!evs) return BNN_OK;
    hipEvent_t e;
    // a timing-only event: no system-scope fence (which would add its own
    // cache writeback to the interval between two kernels)
    HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
    HIP_TRY(hipEventRecord(e, s));
    evs->push_back(e);
    if (label) ops->push_back({label, optype, oe, taps});
    return BNN_OK;
  };
  const bool dump = dmp && dmp->on;
  int pi = 0;  // index into dmp->P
  int rc;
  if ((rc = mark(nullptr, nullptr, 0, 0))) return rc;

  // The forward of patches [nb, nb + cnt) on stream st: the input is
  // [N][bands][H][W], every workspace tensor [N][h][w][words], the logits
  // [N][ncls][H][W], so a part of the batch is the same tensors offset by
  // nb patches.
  int nb = 0, cnt = N;
  hipStream_t st = s;
  auto at = [&](const uint32_t* p, int lvl, int cw) -> const uint32_t* {
    return p ? p + (size_t)nb * hs[lvl] * wsz[lvl] * cw : nullptr;
  };
  auto first_conv = [&]() -> int {
    // v1 enc1.conv1 (3x3) or the v2 stem (1x1): real conv + real fold -> a1 bits
    RealArgs ra{};
    ra.x = sc ? d_in : d_in + (size_t)nb * D->rcin * H * W;  // a scene part moves prow0 instead
    ra.w = D->rw;
    ra.wm = D->rwm;
    ra.alpha = D->ralpha; ra.A = D->rA; ra.B = D->rB; ra.slope = D->rslope; ra.rsign = D->rrsign;
    ra.N = cnt; ra.H = H; ra.W = W; ra.cin = D->rcin; ra.cout = D->rcout;
    ra.out = const_cast<uint32_t*>(at(w.a1, 0, words(D->rcout)));
    ra.f32 = dump ? dmp->conv1 : nullptr;
    if (sc) { ra.sH = sc->sH; ra.sW = sc->sW; ra.pcols = sc->pcols; ra.prow0 = sc->prow0 + nb / sc->pcols; }
    if (D->stem) {
      HIP_TRY(launch_stem(ra, st));
      if ((rc = mark("stem.conv", "conv_real", (double)N * D->rcout * H * W, (double)D->rcin))) return rc;
    } else if (D->cert && real_cert_fits(D->rcin, W, sc ? sc->sW : W) && (uintptr_t)ra.x % 16 == 0) {
      // (the certified kernel stages 16-byte groups; an input that is not
      // 16-byte aligned takes the exact-order kernel below)
      if (dump) {
        RealArgs rf = ra;
        rf.out = nullptr;
        HIP_TRY(launch_real(rf, st));
      }
      ra.f32 = nullptr;
      ra.cwb = D->rcwb;
      ra.cws = D->rcws;
      ra.ct1 = D->rct1; ra.ct2 = D->rct2; ra.cb0 = D->rcb0; ra.cdc = D->rcdc;
      ra.ucnt = D->rcnt;
      HIP_TRY(launch_real_cert(ra, st));
      D->cert_outputs += (unsigned long long)cnt * D->rcout * H * W;
      if ((rc = mark("enc1.conv1", "conv_real", (double)N * D->rcout * H * W, (double)D->rcin * 9))) return rc;
    } else {
      HIP_TRY(launch_real(ra, st));
      if ((rc = mark("enc1.conv1", "conv_real", (double)N * D->rcout * H * W, (double)D->rcin * 9))) return rc;
    }
    return BNN_OK;
  };
  auto bconv = [&](const DevBconv& L, int epi, const uint32_t* in0, const uint32_t* in1, int lvl, int lvl1,
                   uint32_t* out, uint32_t* out2, float* logits, const char* label) -> int {
    BconvArgs a{};
    const int cwo = words(L.cout);
    in0 = at(in0, lvl, L.cw0);
    in1 = at(in1, lvl1, L.cw1);
    out = const_cast<uint32_t*>(at(out, lvl, cwo));
    out2 = const_cast<uint32_t*>(at(out2, lvl + 1, cwo));
    if (logits && !sc) logits += (size_t)nb * D->ncls * H * W;  // a scene part moves prow0 instead
    a.in0 = in0; a.in1 = in1; a.cw0 = L.cw0; a.cw1 = L.cw1;
    a.padoff = 0x80000000u;  // uncovered concat positions read 0 bits
    a.N = cnt; a.H = hs[lvl]; a.W = wsz[lvl]; a.cin = L.cin; a.cout = L.cout;
    if (in1) {
      a.h1 = hs[lvl1]; a.w1 = wsz[lvl1];
      const int uH = 2 * a.h1, uW = 2 * a.w1;
      a.oh = a.H > uH ? (a.H - uH) / 2 : 0;
      a.ow = a.W > uW ? (a.W - uW) / 2 : 0;
      a.uh = std::min(uH, a.H);
      a.uw = std::min(uW, a.W);
    }
    a.wt = L.wt; a.pair = L.pair; a.f1 = L.f1; a.f2 = L.f2;
    a.out = out; a.out2 = out2; a.cwo = words(L.cout);
    a.logits = logits; a.hw = D->hw; a.hb = D->hb; a.ncls = D->ncls;
    if (sc && epi == EPI_HEAD) {
      a.sH = sc->sH; a.sW = sc->sW; a.pcols = sc->pcols; a.prow0 = sc->prow0 + nb / sc->pcols;
    }
    if (dump) {
      a.P = dmp->P[pi++];
      if (epi == EPI_POOL) a.P2 = dmp->P2[lvl];
    }
    const bool mm = use_mfma(L, epi, a.H, a.W);
    if (mm) {
      HIP_TRY(launch_bconv_mfma(a, L.mc, epi, dump, st));
    } else {
      int mt, cog;
      // the shape the whole batch would take: the parts run side by side,
      // so each part's kernel needs only its share of the waves
      pick_shape(epi, N, a.H, a.W, L.cout, &mt, &cog);
      HIP_TRY(launch_bconv(a, epi, mt, cog, dump, st));
    }
    const char* ot = epi == EPI_POOL ? (mm ? "bconv_pool_mfma" : "bconv_pool")
                     : epi == EPI_HEAD ? "bconv_head"
                                       : (mm ? "bconv_mfma" : "bconv");
    return mark(label, ot, (double)N * L.cout * a.H * a.W, (double)L.cin * 9);
  };

  // enc3.c1 .. dec3.c2 as one kernel (level 2 is 8 x 8): input enc2's
  // pooled bits, output dec3.c2's bits; the debug forward takes every
  // intermediate tensor and P as the per-layer kernels would
  const bool use_mid = D->mid && hs[2] == 8 && wsz[2] == 8;
  // and enc2.c1 .. dec2.c2 around it (level 1 is 16 x 16): input enc1's
  // pooled bits, output dec2.c2's bits.  Its blocks run fourteen layers
  // each, one after the other, so it pays only with at least one block per
  // CU (kMidExtMin patches; below that the per-layer kernels, which spread
  // each layer over many more blocks, finish first: 0.123 against 0.132 ms
  // at batch 128).  In a split batch only the last part takes it: the
  // earlier parts' binary layers run beside the next part's first conv,
  // which leaves each CU room for one such block at a time, and the
  // per-layer kernels fill that room better (measured at batch 1024: fused
  // in both parts 0.287 ms, in neither 0.278, in the last 0.268).
  const bool ext_ok = use_mid && D->midx && hs[1] == 16 && wsz[1] == 16;
  bool use_ext = ext_ok && N >= kMidExtMin;
  auto mid = [&]() -> int {
    const auto L = mid_layers(D);
    MidArgs a{};
    double work = 0;
    const DevBconv* XL[kMidXLayers] = {&D->e1[1], &D->e2[1], &D->d1[2], &D->d2[2]};
    auto xlayer = [&](int l) {
      MidXLayer& xl = a.X[l];
      const DevBconv& B = *XL[l];
      xl.w = B.wt;
      xl.lo = B.f1.lo; xl.wid = B.f1.wid;
      xl.lo2 = B.f2.lo; xl.wid2 = B.f2.wid;
      xl.cin = B.cin; xl.cout = B.cout; xl.cw0 = B.cw0; xl.cw1 = B.cw1; xl.pair = B.pair;
      if (dump) {
        xl.P = dmp->P[pi++];
        if (l == 1) xl.P2 = dmp->P2[1];
      }
      work += (double)N * B.cout * 16 * 16 * B.cin * 9;
    };
    if (use_ext) {
      a.ext = 1;
      xlayer(0);
      xlayer(1);
    }
    uint32_t* T[kMidTensors] = {w.down[1], w.h[2], w.skip[2], w.down[2], w.h[3], w.skip[3], w.down[3],
                                w.b1,      w.b2,   w.d1[0],   w.d2[0],   w.d1[1], w.d2[1]};
    static const int lvl[kMidTensors] = {2, 2, 2, 3, 3, 3, 4, 4, 4, 3, 3, 2, 2};
    const int cw[kMidTensors] = {words(D->e2[1].cout), words(L[0]->cout), words(L[1]->cout), words(L[1]->cout),
                                 words(L[2]->cout),    words(L[3]->cout), words(L[3]->cout), words(L[4]->cout),
                                 words(L[5]->cout),    words(L[6]->cout), words(L[7]->cout), words(L[8]->cout),
                                 words(L[9]->cout)};
    for (int l = 0; l < kMidLayers; ++l) {
      MidLayer& ml = a.L[l];
      ml.w = L[l]->mw;
      ml.lo = L[l]->f1.lo; ml.wid = L[l]->f1.wid;
      ml.lo2 = L[l]->f2.lo; ml.wid2 = L[l]->f2.wid;
      ml.cin = L[l]->cin; ml.cout = L[l]->cout;
      if (dump) {
        ml.P = dmp->P[pi++];
        if (l == 1 || l == 3) ml.P2 = dmp->P2[l == 1 ? 2 : 3];
      }
    }
    int off = 0;
    for (int i = 0; i < kMidTensors; ++i) {
      a.t[i] = const_cast<uint32_t*>(at(T[i], lvl[i], cw[i]));
      a.dim[i] = hs[lvl[i]];
      a.cw[i] = cw[i];
      a.off[i] = off;
      off += hs[lvl[i]] * wsz[lvl[i]] * cw[i];
    }
    static const int d[kMidLayers] = {8, 8, 4, 4, 2, 2, 4, 4, 8, 8};
    for (int l = 0; l < kMidLayers; ++l) work += (double)N * L[l]->cout * d[l] * d[l] * L[l]->cin * 9;
    if (use_ext) {
      xlayer(2);
      xlayer(3);
      // 0 enc1 pooled (in), 1 enc2.c1, 2 enc2 skip, 3 dec2.c1, 4 dec2.c2 (out)
      const uint32_t* XT[kMidXTensors] = {w.down[0], w.h[1], w.skip[1], w.d1[2], w.d2[2]};
      const int xcw[kMidXTensors] = {words(D->e2[0].cout), words(D->e1[1].cout), words(D->e2[1].cout),
                                     words(D->d1[2].cout), words(D->d2[2].cout)};
      for (int i = 0; i < kMidXTensors; ++i) {
        a.xt[i] = const_cast<uint32_t*>(at(XT[i], 1, xcw[i]));
        a.xcw[i] = xcw[i];
        a.xoff[i] = off;
        off += 256 * xcw[i];
      }
    }
    a.N = cnt;
    a.ldsw = off;
    HIP_TRY(launch_mid(a, dump, st));
    return mark(use_ext ? "enc2-dec2" : "enc3-dec3", "bconv_mid", work, 1.0);
  };

  static const char* enc_c1[4] = {"enc1.c1", "enc2.c1", "enc3.c1", "enc4.c1"};
  static const char* enc_c2[4] = {"enc1.c2", "enc2.c2", "enc3.c2", "enc4.c2"};
  static const char* dec_c1[4] = {"dec4.c1", "dec3.c1", "dec2.c1", "dec1.c1"};
  static const char* dec_c2[4] = {"dec4.c2", "dec3.c2", "dec2.c2", "dec1.c2"};
  int stage = 3;  // what part() enqueues: 1 the first conv, 2 the binary layers
  auto part = [&]() -> int {
  if ((stage & 1) && (rc = first_conv())) return rc;
  if (!(stage & 2)) return BNN_OK;
  const uint32_t* x = w.a1;
  for (int i = 0; i < (use_ext ? 1 : use_mid ? 2 : 4); ++i) {
    const uint32_t* hin = x;
    if (i || D->stem) {
      if ((rc = bconv(D->e1[i], EPI_FOLD, x, nullptr, i, 0, w.h[i], nullptr, nullptr, enc_c1[i]))) return rc;
      hin = w.h[i];
    }
    if ((rc = bconv(D->e2[i], EPI_POOL, hin, nullptr, i, 0, w.skip[i], w.down[i], nullptr, enc_c2[i]))) return rc;
    x = w.down[i];
  }
  int xl = 4, i0 = 0;
  if (use_mid) {
    if ((rc = mid())) return rc;
    x = use_ext ? w.d2[2] : w.d2[1];
    xl = use_ext ? 1 : 2;
    i0 = use_ext ? 3 : 2;
  } else {
    if ((rc = bconv(D->b1, EPI_FOLD, x, nullptr, 4, 0, w.b1, nullptr, nullptr, "bott.c1"))) return rc;
    if ((rc = bconv(D->b2, EPI_FOLD, w.b1, nullptr, 4, 0, w.b2, nullptr, nullptr, "bott.c2"))) return rc;
    x = w.b2;
  }
  for (int i = i0; i < 4; ++i) {
    const int lvl = 3 - i;
    if ((rc = bconv(D->d1[i], EPI_FOLD, w.skip[lvl], x, lvl, xl, w.d1[i], nullptr, nullptr, dec_c1[i]))) return rc;
    if (i < 3) {
      if ((rc = bconv(D->d2[i], EPI_FOLD, w.d1[i], nullptr, lvl, 0, w.d2[i], nullptr, nullptr, dec_c2[i]))) return rc;
    } else if (D->d2[i].cout > 32) {
      // a head over more than 32 channels: dec1.conv2's bits, then the head
      // on its own (one epilogue group holds at most 32 channels)
      if ((rc = bconv(D->d2[i], EPI_FOLD, w.d1[i], nullptr, lvl, 0, w.d2[i], nullptr, nullptr, dec_c2[i]))) return rc;
      HeadArgs h{};
      h.bits = at(w.d2[i], 0, words(D->d2[i].cout));
      h.cw = words(D->d2[i].cout);
      h.cin = D->d2[i].cout;
      h.hw = D->hw; h.hb = D->hb; h.ncls = D->ncls;
      h.N = cnt; h.H = H; h.W = W;
      h.logits = sc ? d_logits : d_logits + (size_t)nb * D->ncls * H * W;
      if (sc) { h.sH = sc->sH; h.sW = sc->sW; h.pcols = sc->pcols; h.prow0 = sc->prow0 + nb / sc->pcols; }
      HIP_TRY(launch_head_sep(h, st));
      if ((rc = mark("head", "head", (double)N * D->ncls * H * W, (double)h.cin))) return rc;
    } else {
      if ((rc = bconv(D->d2[i], EPI_HEAD, w.d1[i], nullptr, lvl, 0, dump ? w.d2[i] : nullptr, nullptr, d_logits,
                      dec_c2[i])))
        return rc;
    }
    x = w.d2[i];
    xl = lvl;
  }
  return BNN_OK;
  };
  // A large plain batch runs as parts: the binary layers are short and
  // latency bound (launch, ramp and drain are a large part of each kernel),
  // and independent chains keep each other's gaps filled.  Every part's
  // first conv runs on the caller's stream, one after the other (each fills
  // the GPU); a part before the last runs its binary layers on a side stream
  // from the event after its conv, beside the next part's conv, and the last
  // part's layers follow on the caller's stream, which then waits for the
  // side streams.  A forward so begins and ends on the caller's stream, and
  // the next one's first conv follows its last kernel with no wait across
  // streams on the way (with the first conv of the last part on a side
  // stream instead, the wait for it at the end and for the caller's stream
  // at the start left the GPU idle for 17 us a forward at batch 1024).  A
  // scene splits at whole patch rows.  One stream with per-kernel events or
  // debug dumps.
  int parts = 1;
  if (!dump && !evs)
    while (parts < std::min(kSplitMax, max_parts) && N >= kSplitMin * parts * 2) parts *= 2;
  // a scene splits at whole patch rows (its patches are numbered row by row)
  const int unit = sc ? sc->pcols : 1;
  if (sc && N / unit < parts) parts = 1;
  if (parts == 1) return part();
  if (!D->ev_conv[0]) {
    // all or nothing: a failure leaves no half-made set behind
    hipStream_t side[kSplitMax - 1] = {};
    hipEvent_t conv[kSplitMax - 1] = {}, join[kSplitMax - 1] = {};
    // (the conv event orders two streams of this GPU only: the consumer
    // kernels see the conv's output through its own device-scope release,
    // so the event skips the system-scope fence, which cost the caller's
    // stream about 2 us a forward; the join event keeps it, since the
    // caller may read the side streams' logits from the host)
    bool ok = true;
    for (int k = 0; ok && k < kSplitMax - 1; ++k)
      ok = hipStreamCreateWithFlags(&side[k], hipStreamNonBlocking) == hipSuccess &&
           hipEventCreateWithFlags(&conv[k], hipEventDisableTiming | hipEventDisableSystemFence) == hipSuccess &&
           hipEventCreateWithFlags(&join[k], hipEventDisableTiming) == hipSuccess;
    if (!ok) {
      for (int k = 0; k < kSplitMax - 1; ++k) {
        if (conv[k]) (void)hipEventDestroy(conv[k]);
        if (join[k]) (void)hipEventDestroy(join[k]);
        if (side[k]) (void)hipStreamDestroy(side[k]);
      }
      return set_err(BNN_EHIP, "cannot create the streams of a split batch");
    }
    for (int k = 0; k < kSplitMax - 1; ++k) {
      D->side[k] = side[k];
      D->ev_conv[k] = conv[k];
      D->ev_join[k] = join[k];
    }
  }
  const int rows = N / unit;
  // Where two parts meet: at half the batch, or, when the certified first
  // conv runs and the batch is at most one and a half of its rounds (the
  // patches whose blocks it holds at once), after one whole round, so that
  // the second part's conv, at most half a round, splits its patches' rows
  // over two or four blocks and takes a fraction of a round's time
  // (launch_real_cert; config 3's 660 patches as 506 + 154 instead of two
  // half-full rounds of 330)
  long cut = rows / 2;
  if (parts == 2 && !D->stem && D->cert && real_cert_fits(D->rcin, W, sc ? sc->sW : W) &&
      (uintptr_t)d_in % 16 == 0) {
    const long round = real_cert_round(D->rcin, D->rcout, W) / unit;
    if (round > 0 && rows > round && 2 * (rows - round) <= round) cut = round;
  }
  for (int k = 0; k < parts; ++k) {
    nb = parts == 2 ? (int)(k ? cut : 0) * unit : (int)((long)rows * k / parts) * unit;
    cnt = (k + 1 == parts ? N : parts == 2 ? (int)cut * unit : (int)((long)rows * (k + 1) / parts) * unit) - nb;
    use_ext = ext_ok && k + 1 == parts && cnt >= kMidExtMin;
    st = s;
    if (k + 1 == parts) {
      stage = 3;
      if ((rc = part())) return rc;
      break;
    }
    stage = 1;
    if ((rc = part())) return rc;
    HIP_TRY(hipEventRecord(D->ev_conv[k], s));
    HIP_TRY(hipStreamWaitEvent(D->side[k], D->ev_conv[k], 0));
    st = D->side[k];
    stage = 2;
    if ((rc = part())) return rc;
  }
  for (int k = 0; k + 1 < parts; ++k) {
    HIP_TRY(hipEventRecord(D->ev_join[k], D->side[k]));
    HIP_TRY(hipStreamWaitEvent(s, D->ev_join[k], 0));
  }
  return BNN_OK;
}

// The kernels address a launch's tensors with 32-bit byte offsets, so a
// launch covers at most this many patches (its input under 2 GiB, less the
// margin the out-of-range offsets use); larger batches run as several.
int patches_per_launch(const Model* m, int H, int W) {
  const size_t per = (size_t)m->n_bands * H * W * 4;
  return (int)std::min<size_t>(0x7FFFFFF0ull / per, 1u << 30);
}

int check_shape(const Model* m, int N, int H, int W) {
  if (!m || !m->dev) return set_err(BNN_EARG, "model not loaded");
  if (N < 0) return set_err(BNN_EARG, "negative batch");
  if (H < 16 || W < 16)
    return set_err(BNN_EARG, "H=%d W=%d: the four 2x2 pools need H, W >= 16", H, W);
  return BNN_OK;
}

int run_device_launch(const Model* m, const float* d_in, int N, int H, int W, float* d_logits, hipStream_t s,
                      Dumps* dmp);
int grow(float** p, size_t* cap, size_t bytes);

// ------------------------------------------------------------ whole images in tiles
// An image whose input passes the per-launch limit (or, for tests, the tile
// budget BNN_TILE_BYTES) runs as tiles: full-width row strips, or square
// tiles when a strip of 2 * kTileHalo + 16 rows is already too large.  Core
// edges sit on multiples of 16 px, so every 2x2 pool pairs the same rows and
// columns as in the whole image and every inner concat is exact (the
// reference's up_cat offsets, csrc/bnn_model.c:130-148, only arise at the
// image's own bottom and right edges, which a tile ending there shares).
// Each tile runs as an image of its own over its core plus kTileHalo px of
// the image on every side (clipped at the image border); its logits are the
// whole image's on the core.  The zero padding a tile sees at an inner edge
// reaches at most 94 px inward: one row per 3x3 conv at its level, halved
// (rounded up) by each pool, doubled by each upsample -- 2 px after enc1,
// 3, 4, 4 rows after enc2-4, 4 at the bottleneck, then 10, 22, 46 and 94
// after dec4-dec1 (level 3, 2, 1, 0 rows: 8 + 2, 20 + 2, 44 + 2, 92 + 2).
constexpr int kTileHalo = 128;

size_t tile_budget() {
  const char* e = getenv("BNN_TILE_BYTES");
  const size_t def = (size_t)1 << 30;
  if (!e || !*e) return def;
  const long long v = atoll(e);
  return v >= (1 << 20) ? (size_t)v : def;
}

bool needs_tiles(const Model* m, int H, int W) {
  const size_t img = (size_t)m->n_bands * H * W * 4;
  return patches_per_launch(m, H, W) < 1 || img > tile_budget();
}

// core tile sizes (multiples of 16, or the image's own extent)
int plan_tiles(const Model* m, int H, int W, int* th, int* tw) {
  const size_t px = (size_t)m->n_bands * 4, bud = std::min(tile_budget(), (size_t)0x7FFFFFF0ull);
  const size_t rows = bud / (px * W);
  if (rows >= (size_t)2 * kTileHalo + 16) {
    *tw = W;
    *th = (int)std::min<size_t>((rows - 2 * kTileHalo) / 16 * 16, (size_t)H);
    return BNN_OK;
  }
  size_t side = 16;
  while ((side + 16) * (side + 16) * px <= bud) side += 16;
  if (side < (size_t)2 * kTileHalo + 16)
    return set_err(BNN_EARG, "%d bands: a tile of %d px (16 + 2 x %d halo) exceeds the tile budget", m->n_bands,
                   16 + 2 * kTileHalo, kTileHalo);
  *th = *tw = (int)(side - 2 * kTileHalo);
  return BNN_OK;
}

// The tiles of N whole images (input [N][bands][H][W] -> logits
// [N][classes][H][W], host or device pointers) through the staging buffers,
// in order on stream s.
int run_tiles(const Model* m, const float* in, bool in_host, int N, int H, int W, float* out, bool out_host,
              hipStream_t s) {
  int rc, th, tw;
  if ((rc = plan_tiles(m, H, W, &th, &tw))) return rc;
  BnnDevice* D = m->dev;
  const int nb = m->n_bands, nc = m->n_classes;
  const int fh = std::min(H, th + 2 * kTileHalo), fw = std::min(W, tw + 2 * kTileHalo);
  if ((rc = grow(&D->stage_in, &D->stage_in_cap, (size_t)nb * fh * fw * 4))) return rc;
  if ((rc = grow(&D->stage_out, &D->stage_out_cap, (size_t)nc * fh * fw * 4))) return rc;
  const hipMemcpyKind kin = in_host ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice;
  const hipMemcpyKind kout = out_host ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice;
  for (int n = 0; n < N; ++n) {
    const float* img = in + (size_t)n * nb * H * W;
    float* lg = out + (size_t)n * nc * H * W;
    for (int r0 = 0; r0 < H; r0 += th)
      for (int c0 = 0; c0 < W; c0 += tw) {
        const int r1 = std::min(H, r0 + th), c1 = std::min(W, c0 + tw);
        const int a0 = std::max(0, r0 - kTileHalo), a1 = std::min(H, r1 + kTileHalo);
        const int b0 = std::max(0, c0 - kTileHalo), b1 = std::min(W, c1 + kTileHalo);
        const int h = a1 - a0, w = b1 - b0;
        if (h < 16 || w < 16) return set_err(BNN_EARG, "tile %dx%d at (%d, %d): below 16 px", h, w, a0, b0);
        if (w == W) {
          HIP_TRY(hipMemcpy2DAsync(D->stage_in, (size_t)h * W * 4, img + (size_t)a0 * W, (size_t)H * W * 4,
                                   (size_t)h * W * 4, nb, kin, s));
        } else {
          for (int c = 0; c < nb; ++c)
            HIP_TRY(hipMemcpy2DAsync(D->stage_in + (size_t)c * h * w, (size_t)w * 4,
                                     img + (size_t)c * H * W + (size_t)a0 * W + b0, (size_t)W * 4, (size_t)w * 4, h,
                                     kin, s));
        }
        if ((rc = run_device_launch(m, D->stage_in, 1, h, w, D->stage_out, s, nullptr))) return rc;
        for (int c = 0; c < nc; ++c)
          HIP_TRY(hipMemcpy2DAsync(lg + (size_t)c * H * W + (size_t)r0 * W + c0, (size_t)W * 4,
                                   D->stage_out + (size_t)c * h * w + (size_t)(r0 - a0) * w + (c0 - b0),
                                   (size_t)w * 4, (size_t)(c1 - c0) * 4, r1 - r0, kout, s));
      }
  }
  return BNN_OK;
}

int run_device_launch(const Model* m, const float* d_in, int N, int H, int W, float* d_logits, hipStream_t s,
                      Dumps* dmp);

// A batch past the per-launch limit runs as consecutive launches of whole
// sub-batches (the input and logits offset by their first patch), in order
// on the stream.
int run_device(const Model* m, const float* d_in, int N, int H, int W, float* d_logits, hipStream_t s,
               Dumps* dmp) {
  int rc;
  if ((rc = check_shape(m, N, H, W))) return rc;
  if (needs_tiles(m, H, W)) {
    if (dmp && dmp->on) return set_err(BNN_EARG, "a debug forward takes images of at most 2 GiB");
    return run_tiles(m, d_in, false, N, H, W, d_logits, false, s);
  }
  const int per = patches_per_launch(m, H, W);
  if (N > per && dmp && dmp->on) return set_err(BNN_EARG, "a debug forward takes at most %d patches of %dx%d", per, H, W);
  for (int n0 = 0; n0 < N; n0 += per) {
    const int n = std::min(per, N - n0);
    if ((rc = run_device_launch(m, d_in + (size_t)n0 * m->n_bands * H * W, n, H, W,
                                d_logits + (size_t)n0 * m->n_classes * H * W, s, dmp)))
      return rc;
  }
  return BNN_OK;
}

int run_device_launch(const Model* m, const float* d_in, int N, int H, int W, float* d_logits, hipStream_t s,
                      Dumps* dmp) {
  int rc;
  if (N == 0) return BNN_OK;
  BnnDevice* D = m->dev;
  if ((rc = ensure_ws(m, D, D->ws, N, H, W))) return rc;
  if (!g_prof_on) return enqueue_forward(m, D, D->ws, d_in, N, H, W, d_logits, s, dmp, nullptr, nullptr);
  std::vector<Op> ops;
  std::vector<hipEvent_t> evs;
  rc = enqueue_forward(m, D, D->ws, d_in, N, H, W, d_logits, s, dmp, &ops, &evs);
  if (!rc && !evs.empty()) {
    HIP_TRY(hipEventSynchronize(evs.back()));
    for (size_t i = 0; i + 1 < evs.size() && i < ops.size(); ++i) {
      float ms = 0;
      HIP_TRY(hipEventElapsedTime(&ms, evs[i], evs[i + 1]));
      prof_add(ops[i].label, ops[i].optype, ops[i].oe, ops[i].taps, ms * 1e-3);
    }
  }
  for (hipEvent_t e : evs) (void)hipEventDestroy(e);
  return rc;
}

int grow(float** p, size_t* cap, size_t bytes);

// ------------------------------------------------------------ scenes
// Patch-wise scene inference with the tiling of
// csrc/bnn_model_react.c:454-476: P x P patches start at multiples of P, an
// edge patch is zero past the scene, every patch runs as its own image and
// its logits inside the scene go to the map.  The real conv reads the
// patches straight out of the cube and the head writes the map, so no
// patch is ever copied.
int check_scene(const Model* m, int H, int W, int P) {
  if (!m || !m->dev) return set_err(BNN_EARG, "model not loaded");
  if (P < 16 || P % 16) return set_err(BNN_EARG, "patch size %d: must be a positive multiple of 16 (four 2x2 pools)", P);
  if (H < 1 || W < 1) return set_err(BNN_EARG, "scene %dx%d is empty", H, W);
  // one patch row of the cube must fit a launch (strips are whole patch rows)
  if ((size_t)m->n_bands * P * W * 4 >= 0x7FFFFFF0ull)
    return set_err(BNN_EARG, "one row of %dx%d patches of a %d-wide scene exceeds a launch (2 GiB)", P, P, W);
  return BNN_OK;
}

// a cube the kernels can address in place (32-bit byte offsets)
bool scene_in_place(const Model* m, int H, int W) { return (size_t)m->n_bands * H * W * 4 < 0x7FFFFFF0ull; }

// patch rows [prow0, prow0 + nrows) of the scene
int run_scene_rows(const Model* m, const float* d_cube, int H, int W, float* d_map, int P, int prow0, int nrows,
                   hipStream_t s) {
  const int pcols = (W + P - 1) / P;
  const int N = nrows * pcols;
  if (N <= 0) return BNN_OK;
  BnnDevice* D = m->dev;
  int rc;
  if ((rc = ensure_ws(m, D, D->ws, N, P, P))) return rc;
  const Scene sc{H, W, pcols, prow0};
  if (!g_prof_on) return enqueue_forward(m, D, D->ws, d_cube, N, P, P, d_map, s, nullptr, nullptr, nullptr, &sc);
  std::vector<Op> ops;
  std::vector<hipEvent_t> evs;
  rc = enqueue_forward(m, D, D->ws, d_cube, N, P, P, d_map, s, nullptr, &ops, &evs, &sc);
  if (!rc && !evs.empty()) {
    HIP_TRY(hipEventSynchronize(evs.back()));
    for (size_t i = 0; i + 1 < evs.size() && i < ops.size(); ++i) {
      float ms = 0;
      HIP_TRY(hipEventElapsedTime(&ms, evs[i], evs[i + 1]));
      prof_add(ops[i].label, ops[i].optype, ops[i].oe, ops[i].taps, ms * 1e-3);
    }
  }
  for (hipEvent_t e : evs) (void)hipEventDestroy(e);
  return rc;
}

// Scene by strips: R whole patch rows at a time, each staged as its own
// [nb][rows][W] sub-cube (rows = R*P, fewer at the bottom edge) and run as a
// scene of `rows` rows; its map rows [ncls][rows][W] go to the full map with
// one 2-D copy.  Every launch then addresses at most one strip, so cubes of
// any size run, and device memory holds two strips.  A host cube is copied
// through two pinned buffers (host threads fill one while the copy stream
// moves the other and the model's stream runs the strip before); a device
// cube is copied strip by strip on the model's stream.
int run_scene_strips(const Model* m, const float* cube, bool host_cube, int H, int W, float* map, bool host_map,
                     int P, hipStream_t s) {
  int rc;
  if ((rc = check_scene(m, H, W, P))) return rc;
  BnnDevice* D = m->dev;
  const int nb = m->n_bands, ncls = m->n_classes;
  const int prows = (H + P - 1) / P;
  // strips of about 32 MB of input
  const size_t row_bytes = (size_t)nb * P * W * 4;
  const int R = std::max(1, (int)std::min<size_t>(prows, (32u << 20) / row_bytes));
  const size_t strip_bytes = row_bytes * R, smap_bytes = (size_t)ncls * R * P * W * 4;
  for (int k = 0; k < 2; ++k) {
    if ((rc = grow(&D->strip_in[k], &D->strip_in_cap[k], strip_bytes))) return rc;
    if ((rc = grow(&D->strip_out[k], &D->strip_out_cap[k], smap_bytes))) return rc;
  }
  if (host_cube && D->pin_cap < strip_bytes) {
    HIP_TRY(hipDeviceSynchronize());
    for (int k = 0; k < 2; ++k) {
      if (D->pin[k]) (void)hipHostFree(D->pin[k]);
      D->pin[k] = nullptr;
    }
    D->pin_cap = 0;
    for (int k = 0; k < 2; ++k) HIP_TRY(hipHostMalloc((void**)&D->pin[k], strip_bytes, hipHostMallocDefault));
    D->pin_cap = strip_bytes;
  }
  if (!D->copy) {
    HIP_TRY(hipStreamCreateWithFlags(&D->copy, hipStreamNonBlocking));
    for (int k = 0; k < 2; ++k) {
      HIP_TRY(hipEventCreateWithFlags(&D->ev_copied[k], hipEventDisableTiming));
      HIP_TRY(hipEventCreateWithFlags(&D->ev_free[k], hipEventDisableTiming));
      HIP_TRY(hipEventCreateWithFlags(&D->ev_done[k], hipEventDisableTiming));
    }
  }
  const unsigned nthr = std::max(1u, std::min(8u, std::thread::hardware_concurrency()));
  for (int k = 0, pr0 = 0; pr0 < prows; ++k, pr0 += R) {
    const int b = k & 1;
    const int nr = std::min(R, prows - pr0);
    const int r0 = pr0 * P, rows = std::min(nr * P, H - r0);
    const size_t band = (size_t)rows * W;  // floats of one band of the strip
    if (host_cube) {
      if (k >= 2) HIP_TRY(hipEventSynchronize(D->ev_free[b]));  // its copy two strips ago is done
      // [nb][rows][W] of the strip into the pinned buffer, bands split over threads
      float* dst = D->pin[b];
      auto fill = [&](int b0, int b1) {
        for (int c = b0; c < b1; ++c) memcpy(dst + (size_t)c * band, cube + ((size_t)c * H + r0) * W, band * 4);
      };
      std::vector<std::thread> th;
      for (unsigned t = 1; t < nthr; ++t) th.emplace_back(fill, nb * t / nthr, nb * (t + 1) / nthr);
      fill(0, nb / nthr);
      for (auto& t : th) t.join();
      // the strip buffer is free once the strip two before has run
      if (k >= 2) HIP_TRY(hipStreamWaitEvent(D->copy, D->ev_done[b], 0));
      HIP_TRY(hipMemcpyAsync(D->strip_in[b], dst, band * nb * 4, hipMemcpyHostToDevice, D->copy));
      HIP_TRY(hipEventRecord(D->ev_free[b], D->copy));
      HIP_TRY(hipEventRecord(D->ev_copied[b], D->copy));
      HIP_TRY(hipStreamWaitEvent(s, D->ev_copied[b], 0));
    } else {
      HIP_TRY(hipMemcpy2DAsync(D->strip_in[b], band * 4, cube + (size_t)r0 * W, (size_t)H * W * 4, band * 4, nb,
                               hipMemcpyDeviceToDevice, s));
    }
    if ((rc = run_scene_rows(m, D->strip_in[b], rows, W, D->strip_out[b], P, 0, nr, s))) return rc;
    // the strip's map rows span the full width, so each class is one
    // contiguous run of the map; a host map takes plain copies per class
    // (a strided copy into pageable memory lost its order behind the
    // strip's kernels under the profiler's kernel tracing)
    if (host_map) {
      for (int c = 0; c < ncls; ++c)
        HIP_TRY(hipMemcpyAsync(map + ((size_t)c * H + r0) * W, D->strip_out[b] + (size_t)c * band, band * 4,
                               hipMemcpyDeviceToHost, s));
    } else {
      HIP_TRY(hipMemcpy2DAsync(map + (size_t)r0 * W, (size_t)H * W * 4, D->strip_out[b], band * 4, band * 4, ncls,
                               hipMemcpyDeviceToDevice, s));
    }
    HIP_TRY(hipEventRecord(D->ev_done[b], s));
  }
  if (host_map) HIP_TRY(hipStreamSynchronize(s));
  return BNN_OK;
}

// Host cube -> host map, strip by strip.
int run_scene_host(const Model* m, const float* cube, int H, int W, float* map, int P) {
  if (!m || !m->dev) return set_err(BNN_EARG, "model not loaded");
  return run_scene_strips(m, cube, true, H, W, map, true, P, m->dev->stream);
}

int grow(float** p, size_t* cap, size_t bytes) {
  if (*cap >= bytes) return BNN_OK;
  if (*p) { HIP_TRY(hipDeviceSynchronize()); (void)hipFree(*p); }
  *p = nullptr;
  *cap = 0;
  HIP_TRY(hipMalloc((void**)p, bytes));
  *cap = bytes;
  return BNN_OK;
}

// Host input -> host logits, in sub-batches of at most one launch each
// (staging buffers of one sub-batch, so device memory stays bounded).
int run_host(const Model* m, const float* input, int N, int H, int W, float* logits, Dumps* dmp) {
  int rc;
  if ((rc = check_shape(m, N, H, W))) return rc;
  if (N == 0) return BNN_OK;
  BnnDevice* D = m->dev;
  if (needs_tiles(m, H, W)) {
    if (dmp && dmp->on) return set_err(BNN_EARG, "a debug forward takes images of at most 2 GiB");
    if ((rc = run_tiles(m, input, true, N, H, W, logits, true, D->stream))) return rc;
    HIP_TRY(hipStreamSynchronize(D->stream));
    return BNN_OK;
  }
  const int per = patches_per_launch(m, H, W);
  if (N > per && dmp && dmp->on) return set_err(BNN_EARG, "a debug forward takes at most %d patches of %dx%d", per, H, W);
  const int nc = std::min(N, per);
  const size_t pin = (size_t)m->n_bands * H * W * 4, pout = (size_t)m->n_classes * H * W * 4;
  if ((rc = grow(&D->stage_in, &D->stage_in_cap, pin * nc))) return rc;
  if ((rc = grow(&D->stage_out, &D->stage_out_cap, pout * nc))) return rc;
  for (int n0 = 0; n0 < N; n0 += nc) {
    const int n = std::min(nc, N - n0);
    HIP_TRY(hipMemcpyAsync(D->stage_in, (const char*)input + pin * n0, pin * n, hipMemcpyHostToDevice, D->stream));
    if ((rc = run_device_launch(m, D->stage_in, n, H, W, D->stage_out, D->stream, dmp))) return rc;
    HIP_TRY(hipMemcpyAsync((char*)logits + pout * n0, D->stage_out, pout * n, hipMemcpyDeviceToHost, D->stream));
  }
  HIP_TRY(hipStreamSynchronize(D->stream));
  return BNN_OK;
}

}  // namespace

// =================================================================== C ABI
extern "C" {

const char* bnn_last_error(void) { return g_err.c_str(); }

int bnn_blob_check(const char* path) {
  Model* m = nullptr;
  int rc = parse_blob(path, &m);
  if (rc) return rc;
  rc = validate(m);
  free_host(m);
  free(m);
  return rc;
}

void bnn_free(Model* m) {
  if (!m) return;
  if (m->dev) {
    release(m->dev);
    delete m->dev;
    m->dev = nullptr;
  }
  free_host(m);
  free(m);
}

int bnn_load_status(const char* path, Model** out) {
  *out = nullptr;
  Model* m = nullptr;
  int rc = parse_blob(path, &m);
  if (rc) return rc;
  if ((rc = validate(m)) || (rc = build_device(m))) {
    const std::string keep = g_err;
    bnn_free(m);
    g_err = keep;
    return rc;
  }
  *out = m;
  return BNN_OK;
}

Model* bnn_load(const char* path) {
  Model* m = nullptr;
  if (bnn_load_status(path, &m)) die();
  return m;
}

int bnn_forward_batch(const Model* m, const float* input, int N, int H, int W, float* logits) {
  return run_host(m, input, N, H, W, logits, nullptr);
}

void bnn_forward(const Model* m, const float* input, int H, int W, float* logits) {
  prof_reset();
  if (bnn_forward_batch(m, input, 1, H, W, logits)) die();
}

int bnn_forward_device(const Model* m, const float* d_input, int N, int H, int W, float* d_logits,
                       void* stream) {
  return run_device(m, d_input, N, H, W, d_logits, (hipStream_t)stream, nullptr);
}

void* bnn_stream(const Model* m) { return (m && m->dev) ? (void*)m->dev->stream : nullptr; }

int bnn_forward_device_noalloc(const Model* m, const float* d_input, int N, int H, int W, float* d_logits,
                               void* stream) {
  int rc;
  if ((rc = check_shape(m, N, H, W))) return rc;
  if (N == 0) return BNN_OK;
  BnnDevice* D = m->dev;
  if (!D->scratch) return set_err(BNN_EHIP, "allocation-free forward unavailable: %s", D->scratch_err.c_str());
  // sub-batches of at most patches_per_launch, as run_device splits them
  const int per = patches_per_launch(m, H, W);
  if (per < 1)
    return set_err(BNN_EARG, "one %dx%d image of %d bands exceeds a launch (2 GiB): it runs in tiles through "
                   "staging buffers, which the allocation-free forward does not allocate", H, W, m->n_bands);
  Workspace w;
  const size_t need = plan_ws(m, D, w, std::min(N, per), H, W, nullptr);
  if (need > (size_t)BNN_NOALLOC_SCRATCH_BYTES)
    return set_err(BNN_EARG, "N=%d H=%d W=%d needs %zu bytes of scratch; the allocation-free forward holds %zu",
                   N, H, W, need, (size_t)BNN_NOALLOC_SCRATCH_BYTES);
  for (int n0 = 0; n0 < N; n0 += per) {
    const int n = std::min(per, N - n0);
    plan_ws(m, D, w, n, H, W, D->scratch);
    // one part on the caller's stream: no side streams, events or profiling
    if ((rc = enqueue_forward(m, D, w, d_input + (size_t)n0 * m->n_bands * H * W, n, H, W,
                              d_logits + (size_t)n0 * m->n_classes * H * W, (hipStream_t)stream, nullptr, nullptr,
                              nullptr, nullptr, 1)))
      return rc;
  }
  return BNN_OK;
}

int bnn_forward_patched(const Model* m, const float* input, int H, int W, float* logits, int P) {
  return run_scene_host(m, input, H, W, logits, P);
}

int bnn_forward_patched_device(const Model* m, const float* d_input, int H, int W, float* d_logits, int P,
                               void* stream) {
  int rc;
  if ((rc = check_scene(m, H, W, P))) return rc;
  // in place when the kernels can address the cube, else strip by strip
  if (scene_in_place(m, H, W))
    return run_scene_rows(m, d_input, H, W, d_logits, P, 0, (H + P - 1) / P, (hipStream_t)stream);
  return run_scene_strips(m, d_input, false, H, W, d_logits, false, P, (hipStream_t)stream);
}

int bnn_forward_debug(const Model* m, const float* input, int N, int H, int W, float* logits, bnn_stage_cb cb,
                      void* ctx) {
  int rc;
  if ((rc = check_shape(m, N, H, W))) return rc;
  if (N == 0) return BNN_OK;
  BnnDevice* D = m->dev;
  int hs[5], ws[5];
  level_dims(H, W, hs, ws);
  // P dumps in launch order, with the (c, level) of each
  struct PInfo { const char* name; int c, lvl; };
  std::vector<PInfo> pinfo;
  if (D->stem) pinfo.push_back({"enc1.conv1.P", m->enc_conv1[0].Cout, 0});
  pinfo.push_back({"enc1.conv2.P", m->enc_conv2[0].Cout, 0});
  static const char* encn[4][2] = {{"", "enc1.conv2.P"}, {"enc2.conv1.P", "enc2.conv2.P"},
                                   {"enc3.conv1.P", "enc3.conv2.P"}, {"enc4.conv1.P", "enc4.conv2.P"}};
  for (int i = 1; i < 4; ++i) {
    pinfo.push_back({encn[i][0], m->enc_conv1[i].Cout, i});
    pinfo.push_back({encn[i][1], m->enc_conv2[i].Cout, i});
  }
  pinfo.push_back({"bott.conv1.P", m->bott_conv1.Cout, 4});
  pinfo.push_back({"bott.conv2.P", m->bott_conv2.Cout, 4});
  static const char* decn[4][2] = {{"dec4.conv1.P", "dec4.conv2.P"}, {"dec3.conv1.P", "dec3.conv2.P"},
                                   {"dec2.conv1.P", "dec2.conv2.P"}, {"dec1.conv1.P", "dec1.conv2.P"}};
  for (int i = 0; i < 4; ++i) {
    pinfo.push_back({decn[i][0], m->dec_conv1[i].Cout, 3 - i});
    pinfo.push_back({decn[i][1], m->dec_conv2[i].Cout, 3 - i});
  }
  Dumps d;
  d.on = true;
  std::vector<void*> tmp;
  bool oom = false;  // any failed allocation: no dump kernel may run with a null target
  auto alloc = [&](size_t bytes) -> void* {
    void* p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 4) != hipSuccess) {
      (void)hipGetLastError();
      oom = true;
      return nullptr;
    }
    tmp.push_back(p);
    return p;
  };
  auto cleanup = [&]() { for (void* p : tmp) (void)hipFree(p); };
  d.conv1 = (float*)alloc((size_t)N * D->rcout * H * W * 4);
  for (size_t i = 0; i < pinfo.size(); ++i)
    d.P[i] = (int32_t*)alloc((size_t)N * pinfo[i].c * hs[pinfo[i].lvl] * ws[pinfo[i].lvl] * 4);
  for (int i = 0; i < 4; ++i) d.P2[i] = (int32_t*)alloc((size_t)N * m->enc_conv2[i].Cout * hs[i + 1] * ws[i + 1] * 4);
  if (oom) { cleanup(); return set_err(BNN_EHIP, "hipMalloc failed for debug dumps (N=%d)", N); }
  if ((rc = run_host(m, input, N, H, W, logits, &d))) { cleanup(); return rc; }
  if (cb) {
    const Workspace& w = D->ws;
    auto emit_f = [&](const char* name, const void* dptr, int dtype, int c, int lvl) -> int {
      const size_t n = (size_t)N * c * hs[lvl] * ws[lvl];
      std::vector<uint8_t> h(n * 4);
      HIP_TRY(hipMemcpy(h.data(), dptr, n * 4, hipMemcpyDeviceToHost));
      cb(ctx, name, dtype, N, c, hs[lvl], ws[lvl], h.data());
      return BNN_OK;
    };
    // packed bits [N][h][w][cw] -> int8 +-1 [N][c][h][w]
    auto emit_b = [&](const char* name, const uint32_t* dptr, int c, int lvl) -> int {
      const int hh = hs[lvl], ww = ws[lvl], cw = words(c);
      const size_t np = (size_t)N * hh * ww;
      std::vector<uint32_t> pk(np * cw);
      HIP_TRY(hipMemcpy(pk.data(), dptr, pk.size() * 4, hipMemcpyDeviceToHost));
      std::vector<int8_t> out((size_t)N * c * hh * ww);
      for (int n = 0; n < N; ++n)
        for (int ch = 0; ch < c; ++ch)
          for (int p = 0; p < hh * ww; ++p) {
            const uint32_t word = pk[((size_t)n * hh * ww + p) * cw + (ch >> 5)];
            out[((size_t)n * c + ch) * hh * ww + p] = ((word >> (ch & 31)) & 1u) ? 1 : -1;
          }
      cb(ctx, name, 0, N, c, hh, ww, out.data());
      return BNN_OK;
    };
    char nm[48];
    int pi = 0;
    if ((rc = emit_f(D->stem ? "stem.conv" : "enc1.conv1", d.conv1, 2, D->rcout, 0))) goto done;
    if ((rc = emit_b(D->stem ? "stem.act" : "enc1.act1", w.a1, D->rcout, 0))) goto done;
    for (int i = 0; i < 4; ++i) {
      if (i || D->stem) {
        if ((rc = emit_f(pinfo[pi].name, d.P[pi], 1, pinfo[pi].c, i))) goto done;
        ++pi;
        snprintf(nm, sizeof nm, "enc%d.act1", i + 1);
        if ((rc = emit_b(nm, w.h[i], m->enc_conv1[i].Cout, i))) goto done;
      }
      if ((rc = emit_f(pinfo[pi].name, d.P[pi], 1, pinfo[pi].c, i))) goto done;
      ++pi;
      snprintf(nm, sizeof nm, "enc%d.act2_skip", i + 1);
      if ((rc = emit_b(nm, w.skip[i], m->enc_conv2[i].Cout, i))) goto done;
      snprintf(nm, sizeof nm, "enc%d.pool.P", i + 1);
      if ((rc = emit_f(nm, d.P2[i], 1, m->enc_conv2[i].Cout, i + 1))) goto done;
      snprintf(nm, sizeof nm, "enc%d.act2_down", i + 1);
      if ((rc = emit_b(nm, w.down[i], m->enc_conv2[i].Cout, i + 1))) goto done;
    }
    if ((rc = emit_f(pinfo[pi].name, d.P[pi], 1, pinfo[pi].c, 4))) goto done;
    ++pi;
    if ((rc = emit_b("bott.act1", w.b1, m->bott_conv1.Cout, 4))) goto done;
    if ((rc = emit_f(pinfo[pi].name, d.P[pi], 1, pinfo[pi].c, 4))) goto done;
    ++pi;
    if ((rc = emit_b("bott.act2", w.b2, m->bott_conv2.Cout, 4))) goto done;
    for (int i = 0; i < 4; ++i) {
      const int lvl = 3 - i;
      if ((rc = emit_f(pinfo[pi].name, d.P[pi], 1, pinfo[pi].c, lvl))) goto done;
      ++pi;
      snprintf(nm, sizeof nm, "dec%d.act1", 4 - i);
      if ((rc = emit_b(nm, w.d1[i], m->dec_conv1[i].Cout, lvl))) goto done;
      if ((rc = emit_f(pinfo[pi].name, d.P[pi], 1, pinfo[pi].c, lvl))) goto done;
      ++pi;
      snprintf(nm, sizeof nm, "dec%d.act2", 4 - i);
      if ((rc = emit_b(nm, w.d2[i], m->dec_conv2[i].Cout, lvl))) goto done;
    }
    cb(ctx, "logits", 2, N, m->n_classes, H, W, logits);
  }
done:
  cleanup();
  return rc;
}

// =========================================================== v2 stem C ABI
}  // extern "C"

namespace {
// A StemModel handed out by bnn_stem_load is the first member of this holder;
// `body` is the same network seen as a Model (the stem's records aside, the
// v2 body has v1's records in v1's order), sharing the host arrays, so the
// v1 machinery runs it with the device model's stem flag set.
struct StemHolder {
  StemModel pub;
  Model body;
  StemPart st;
};
static_assert(offsetof(StemHolder, pub) == 0, "StemModel must be the holder's first member");
static_assert(sizeof(ConvS) == sizeof(Conv) && sizeof(ActS) == sizeof(Act), "v1 and v2 records differ");

const Model* body_of(const StemModel* m) {
  return m ? &reinterpret_cast<const StemHolder*>(m)->body : nullptr;
}

void stem_public(StemHolder* h) {
  StemModel& p = h->pub;
  const Model& b = h->body;
  p.version = b.version; p.base_channels = b.base_channels;
  p.n_bands = b.n_bands; p.n_classes = b.n_classes; p.upsampler = b.upsampler;
  p.has_stem = h->st.has_stem; p.n_stem_layers = h->st.n_stem_layers;
  memcpy(&p.stem_conv, &h->st.c, sizeof(Conv));
  memcpy(&p.stem_act, &h->st.a, sizeof(Act));
  for (int i = 0; i < 4; ++i) {
    memcpy(&p.enc_conv1[i], &b.enc_conv1[i], sizeof(Conv)); memcpy(&p.enc_conv2[i], &b.enc_conv2[i], sizeof(Conv));
    memcpy(&p.enc_act1[i], &b.enc_act1[i], sizeof(Act));
    memcpy(&p.enc_act2_skip[i], &b.enc_act2_skip[i], sizeof(Act));
    memcpy(&p.enc_act2_down[i], &b.enc_act2_down[i], sizeof(Act));
    memcpy(&p.dec_conv1[i], &b.dec_conv1[i], sizeof(Conv)); memcpy(&p.dec_conv2[i], &b.dec_conv2[i], sizeof(Conv));
    memcpy(&p.dec_act1[i], &b.dec_act1[i], sizeof(Act)); memcpy(&p.dec_act2[i], &b.dec_act2[i], sizeof(Act));
  }
  memcpy(&p.bott_conv1, &b.bott_conv1, sizeof(Conv)); memcpy(&p.bott_conv2, &b.bott_conv2, sizeof(Conv));
  memcpy(&p.bott_act1, &b.bott_act1, sizeof(Act)); memcpy(&p.bott_act2, &b.bott_act2, sizeof(Act));
  p.head_Cout = b.head_Cout; p.head_Cin = b.head_Cin;
  p.head_W = b.head_W; p.head_bias = b.head_bias;
  p.dev = b.dev;
}
}  // namespace

extern "C" {

int bnn_stem_blob_check(const char* path) {
  Model* m = nullptr;
  StemPart st;
  int rc = parse_blob(path, &m, 2, &st);
  if (rc) return rc;
  rc = validate(m, &st);
  free_host(m);
  free(m);
  free_conv(&st.c);
  free_act(&st.a);
  return rc;
}

void bnn_stem_free(StemModel* sm) {
  if (!sm) return;
  StemHolder* h = reinterpret_cast<StemHolder*>(sm);
  if (h->body.dev) {
    release(h->body.dev);
    delete h->body.dev;
    h->body.dev = nullptr;
  }
  free_host(&h->body);
  free_conv(&h->st.c);
  free_act(&h->st.a);
  free(h);
}

int bnn_stem_load_status(const char* path, StemModel** out) {
  *out = nullptr;
  Model* m = nullptr;
  StemPart st;
  int rc = parse_blob(path, &m, 2, &st);
  if (rc) return rc;
  StemHolder* h = (StemHolder*)calloc(1, sizeof(StemHolder));
  if (!h) {
    free_host(m); free(m); free_conv(&st.c); free_act(&st.a);
    return set_err(BNN_EBLOB, "out of memory");
  }
  h->body = *m;  // takes over the arrays
  free(m);
  h->st = st;
  if ((rc = validate(&h->body, &h->st)) || (rc = build_device(&h->body, &h->st))) {
    const std::string keep = g_err;
    bnn_stem_free(&h->pub);
    g_err = keep;
    return rc;
  }
  stem_public(h);
  *out = &h->pub;
  return BNN_OK;
}

StemModel* bnn_stem_load(const char* path) {
  StemModel* m = nullptr;
  if (bnn_stem_load_status(path, &m)) die();
  return m;
}

int bnn_stem_forward_batch(const StemModel* m, const float* input, int N, int H, int W, float* logits) {
  return run_host(body_of(m), input, N, H, W, logits, nullptr);
}

void bnn_stem_forward(const StemModel* m, const float* input, int H, int W, float* logits) {
  prof_reset();
  if (bnn_stem_forward_batch(m, input, 1, H, W, logits)) die();
}

int bnn_stem_forward_device(const StemModel* m, const float* d_input, int N, int H, int W, float* d_logits,
                            void* stream) {
  return run_device(body_of(m), d_input, N, H, W, d_logits, (hipStream_t)stream, nullptr);
}

void* bnn_stem_stream(const StemModel* m) { return bnn_stream(body_of(m)); }

int bnn_stem_forward_patched(const StemModel* m, const float* input, int H, int W, float* logits, int P) {
  return bnn_forward_patched(body_of(m), input, H, W, logits, P);
}

int bnn_stem_forward_patched_device(const StemModel* m, const float* d_input, int H, int W, float* d_logits,
                                    int P, void* stream) {
  return bnn_forward_patched_device(body_of(m), d_input, H, W, d_logits, P, stream);
}

int bnn_stem_forward_debug(const StemModel* m, const float* input, int N, int H, int W, float* logits,
                           bnn_stem_stage_cb cb, void* ctx) {
  return bnn_forward_debug(body_of(m), input, N, H, W, logits, cb, ctx);
}

// ----------------------------------------------------------- profiler API
double prof_now(void) {
  struct timespec t;
  clock_gettime(CLOCK_MONOTONIC, &t);
  return (double)t.tv_sec + (double)t.tv_nsec * 1e-9;
}
void prof_reset(void) { g_prof.clear(); }
void prof_add(const char* label, const char* optype, double out_elems, double taps, double sec) {
  if (g_prof.size() >= 65536) return;
  g_prof.push_back({label ? label : "?", optype ? optype : "?", out_elems, taps, sec});
}
void prof_report(FILE* o) {
  if (g_prof.empty()) return;
  double tot = 0;
  for (auto& r : g_prof) tot += r.sec;
  auto work = [](const ProfRec& r) { return r.oe * (r.taps > 0 ? r.taps : 1.0); };
  fprintf(o, "\n# per-op (execution order, GPU kernel time)\n");
  fprintf(o, "%-14s %-10s %12s %12s %10s %7s\n", "layer", "op", "out_elems", "work", "ms", "%");
  for (auto& r : g_prof)
    fprintf(o, "%-14s %-10s %12.0f %12.4g %10.4f %6.2f\n", r.label.c_str(), r.optype.c_str(), r.oe, work(r),
            r.sec * 1e3, tot > 0 ? 100.0 * r.sec / tot : 0.0);
  fprintf(o, "\n# roll-up by op type\n");
  fprintf(o, "%-10s %6s %12s %10s %7s\n", "op", "calls", "work", "ms", "%");
  std::vector<std::string> seen;
  for (auto& r : g_prof)
    if (std::find(seen.begin(), seen.end(), r.optype) == seen.end()) seen.push_back(r.optype);
  for (auto& t : seen) {
    double s = 0, w = 0;
    int c = 0;
    for (auto& r : g_prof)
      if (r.optype == t) { s += r.sec; w += work(r); ++c; }
    fprintf(o, "%-10s %6d %12.4g %10.4f %6.2f\n", t.c_str(), c, w, s * 1e3, tot > 0 ? 100.0 * s / tot : 0.0);
  }
  fprintf(o, "# total per-op: %.4f ms\n", tot * 1e3);
}
int bnn_cert_stats(const Model* m, unsigned long long* undecided, unsigned long long* outputs) {
  if (!m || !m->dev) return set_err(BNN_EARG, "model not loaded");
  BnnDevice* D = m->dev;
  unsigned long long u = 0;
  if (D->rcnt) {
    HIP_TRY(hipSetDevice(D->device));
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipMemcpy(&u, D->rcnt, sizeof u, hipMemcpyDeviceToHost));
    HIP_TRY(hipMemset(D->rcnt, 0, sizeof u));
  }
  if (undecided) *undecided = u;
  if (outputs) *outputs = D->cert_outputs;
  D->cert_outputs = 0;
  return BNN_OK;
}

void bnn_prof_enable(int on) { g_prof_on = on != 0; }
int bnn_prof_count(void) { return (int)g_prof.size(); }
int bnn_prof_get(int i, char* label, int label_len, char* optype, int optype_len, double* ms, double* work) {
  if (i < 0 || i >= (int)g_prof.size()) return set_err(BNN_EARG, "profile index out of range");
  const ProfRec& r = g_prof[i];
  if (label && label_len > 0) snprintf(label, label_len, "%s", r.label.c_str());
  if (optype && optype_len > 0) snprintf(optype, optype_len, "%s", r.optype.c_str());
  if (ms) *ms = r.sec * 1e3;
  if (work) *work = r.oe * (r.taps > 0 ? r.taps : 1.0);
  return BNN_OK;
}

// ------------------------------------------------------------ fold canon
void bnn_fold_canon(const int32_t* type, const int32_t* t, const int32_t* lo, const int32_t* hi, int C,
                    int32_t* out_lo, uint32_t* out_wid, uint8_t* out_inv) {
  // |P| <= Cin*9 < 2^30, so clamping thresholds to +-2^30 changes no decision
  // and keeps P - lo free of overflow.
  const int32_t L = 1 << 30;
  auto cl = [&](int32_t v) { return v < -L ? -L : (v > L ? L : v); };
  for (int c = 0; c < C; ++c) {
    int32_t l = 0;
    uint32_t w = 0;
    uint8_t inv = 0;
    switch (type[c]) {
      case 0: inv = t[c] > 0; break;                                  // constant
      case 1: l = cl(t[c]); w = 0x80000000u; break;                   // P >= t
      case 2: l = cl(t[c]); w = 0x80000000u; inv = 1; break;          // P <  t
      case 3:                                                         // lo <= P < hi
      case 4: {                                                       // P < lo || P >= hi
        const int32_t a = cl(lo[c]), b = cl(hi[c]);
        if (a < b) { l = a; w = (uint32_t)(b - a); }
        inv = type[c] == 4;
        break;
      }
      default: break;                                                 // -1 everywhere
    }
    out_lo[c] = l;
    out_wid[c] = w;
    out_inv[c] = inv;
  }
}

// ------------------------------------------------------- isolated layers
BnnConvLayer* bnn_layer_create(const uint64_t* packed_w, int Cin, int Cout, const int32_t* type1,
                               const int32_t* t1, const int32_t* lo1, const int32_t* hi1, const int32_t* type2,
                               const int32_t* t2, const int32_t* lo2, const int32_t* hi2) {
  if (Cin <= 0 || Cout <= 0 || !packed_w) { set_err(BNN_EARG, "bad layer shape"); return nullptr; }
  BnnConvLayer* Lr = new BnnConvLayer();
  BnnDevice* D = &Lr->dev;
  auto fail = [&]() -> BnnConvLayer* { release(D); delete Lr; return nullptr; };
  if (hipGetDevice(&D->device) != hipSuccess) { set_err(BNN_EHIP, "no HIP device"); return fail(); }
  if (hipStreamCreateWithFlags(&D->stream, hipStreamNonBlocking) != hipSuccess) {
    set_err(BNN_EHIP, "hipStreamCreate failed");
    return fail();
  }
  Conv c{};
  c.tag = TAG_BIN; c.Cin = Cin; c.Cout = Cout; c.kh = c.kw = 3; c.pad = c.stride = 1;
  c.nwords = (Cin * 9 + 63) / 64;
  c.packed = const_cast<uint64_t*>(packed_w);
  Act a1{}, a2{};
  a1.C = a2.C = Cout;
  a1.type = const_cast<int32_t*>(type1); a1.t = const_cast<int32_t*>(t1);
  a1.lo = const_cast<int32_t*>(lo1); a1.hi = const_cast<int32_t*>(hi1);
  a2.type = const_cast<int32_t*>(type2); a2.t = const_cast<int32_t*>(t2);
  a2.lo = const_cast<int32_t*>(lo2); a2.hi = const_cast<int32_t*>(hi2);
  if (upload_bconv(D, &Lr->L, c, 0, type1 ? &a1 : nullptr, type2 ? &a2 : nullptr)) return fail();
  return Lr;
}

void bnn_layer_free(BnnConvLayer* L) {
  if (!L) return;
  release(&L->dev);
  delete L;
}

static int layer_args(const BnnConvLayer* L, const uint32_t* d_act, int N, int H, int W, BconvArgs* a) {
  if (!L) return set_err(BNN_EARG, "null layer");
  if (N < 0 || H <= 0 || W <= 0) return set_err(BNN_EARG, "bad shape");
  *a = BconvArgs{};
  a->in0 = d_act; a->cw0 = L->L.cw0; a->N = N; a->H = H; a->W = W;
  a->cin = L->L.cin; a->cout = L->L.cout; a->wt = L->L.wt; a->pair = L->L.pair; a->f1 = L->L.f1; a->f2 = L->L.f2;
  a->cwo = words(L->L.cout);
  return BNN_OK;
}

int bnn_layer_P_device(const BnnConvLayer* L, const uint32_t* d_act, int N, int H, int W, int32_t* d_P,
                       void* stream) {
  BconvArgs a;
  int rc;
  if ((rc = layer_args(L, d_act, N, H, W, &a))) return rc;
  a.P = d_P;
  int mt, cog;
  pick_shape(EPI_P, N, H, W, a.cout, &mt, &cog);
  HIP_TRY(launch_bconv(a, EPI_P, mt, cog, false, (hipStream_t)stream));
  return BNN_OK;
}

int bnn_layer_fold_pool_device(const BnnConvLayer* L, const uint32_t* d_act, int N, int H, int W,
                               uint32_t* d_skip, uint32_t* d_down, void* stream) {
  BconvArgs a;
  int rc;
  if ((rc = layer_args(L, d_act, N, H, W, &a))) return rc;
  if (!L->L.f1.lo || !L->L.f2.lo) return set_err(BNN_EARG, "layer was created without both rules");
  if (H < 2 || W < 2) return set_err(BNN_EARG, "pool needs H, W >= 2");
  a.out = d_skip; a.out2 = d_down;
  if (use_mfma(L->L, EPI_POOL, H, W)) {
    HIP_TRY(launch_bconv_mfma(a, L->L.mc, EPI_POOL, false, (hipStream_t)stream));
    return BNN_OK;
  }
  int mt, cog;
  pick_shape(EPI_POOL, N, H, W, a.cout, &mt, &cog);
  HIP_TRY(launch_bconv(a, EPI_POOL, mt, cog, false, (hipStream_t)stream));
  return BNN_OK;
}

int bnn_pack_act_device(const int8_t* d_a, uint32_t* d_out, int N, int C, int H, int W, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  HIP_TRY(launch_pack_act(d_a, d_out, N, C, H, W, s));
  return BNN_OK;
}

}  // extern "C"
