/* bnn_model_stem.h - C ABI of libbnn_hip.so for the v2 (spectral-stem)
 * model: a real-input 1x1 binary-weight stem with a real fold, then the v1
 * body with enc1.conv1 binary.
 *
 * Drop-in for the reference's csrc/bnn_model_stem.h: the same record types
 * (ConvS/ActS), the same StemModel field order (plus a trailing device
 * pointer, as Model has in bnn_model.h), and bnn_stem_load / bnn_stem_free /
 * bnn_stem_forward with the reference's argument meaning and error
 * behaviour (message on stderr, exit(1)).  The same library serves both
 * headers; the error codes, bnn_last_error(), the profiler and the kernel
 * entry points are the ones declared in bnn_model.h.
 */
#ifndef BNN_MODEL_STEM_H
#define BNN_MODEL_STEM_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- shared kernels: csrc/bnn_model_stem.h:14-25 (one definition each,
 * also declared in bnn_model.h) ---- */
void bconv_dispatch(const int8_t *a, const uint64_t *packed_w, int32_t *P,
                int Cin, int H, int W, int Cout, int kh, int kw, int pad, int stride);
void conv_realin_naive(const float *x, const int8_t *wsign, const float *alpha,
                       float *out, int Cin, int H, int W, int Cout,
                       int kh, int kw, int pad, int stride);
void maxpool_P(const int32_t *P, int32_t *Pout, int C, int H, int W, int k, int stride);
void apply_fold_int(const int32_t *P, int8_t *out, int C, int H, int W,
                    const int32_t *type, const int32_t *t, const int32_t *lo, const int32_t *hi);
void apply_fold_real(const float *x, int8_t *out, int C, int H, int W,
                     const float *A, const float *B, const float *slope, const float *rsign);
void head_1x1(const float *a, const float *W, const float *bias,
              float *logits, int Cin, int H, int W_, int Cout);

/* ---- parsed blob records: csrc/bnn_model_stem.h:27-42 ---- */
typedef struct {
    int tag;                 /* 1 = binary (packed), 2 = real (wsign+alpha) */
    int Cout, Cin, kh, kw, pad, stride, nwords;
    uint64_t *packed;
    int8_t *wsign;
    float *alpha;
} ConvS;

typedef struct {
    int kind;                /* 0 = integer-P fold, 1 = real fold */
    int C;
    int32_t *type, *t, *lo, *hi;
    float *A, *B, *slope, *rsign;
} ActS;

struct BnnDevice;

/* ---- csrc/bnn_model_stem.h:44-59 ---- */
typedef struct {
    int version, base_channels, n_bands, n_classes, upsampler;
    int has_stem, n_stem_layers;   /* v2: has_stem==1, n_stem_layers==1 */
    ConvS stem_conv;               /* real-input binary-weight 1x1 conv */
    ActS  stem_act;                /* real fold */
    ConvS enc_conv1[4], enc_conv2[4];   /* enc1.conv1 is binary here */
    ActS  enc_act1[4], enc_act2_skip[4], enc_act2_down[4];
    ConvS bott_conv1, bott_conv2;
    ActS  bott_act1, bott_act2;
    ConvS dec_conv1[4], dec_conv2[4];
    ActS  dec_act1[4], dec_act2[4];
    int head_Cout, head_Cin;
    float *head_W, *head_bias;
    struct BnnDevice *dev;   /* not in the reference; owned by the library */
} StemModel;

/* ---- csrc/bnn_model_stem.h:61-64 ---- */
StemModel *bnn_stem_load(const char *path);   /* never NULL: exits(1) on any error */
void bnn_stem_free(StemModel *m);
/* input: [n_bands, H, W] float; logits: [n_classes, H, W] float (caller allocs) */
void bnn_stem_forward(const StemModel *m, const float *input, int H, int W, float *logits);

/* ---- extensions (no counterpart in the reference), the v2 twins of the
 * bnn_model.h extensions of the same names without "_stem" ---- */
int bnn_stem_blob_check(const char *path);
int bnn_stem_load_status(const char *path, StemModel **out);
int bnn_stem_forward_batch(const StemModel *m, const float *input, int N, int H, int W, float *logits);
int bnn_stem_forward_device(const StemModel *m, const float *d_input, int N, int H, int W,
                            float *d_logits, void *stream);
void *bnn_stem_stream(const StemModel *m);
int bnn_stem_forward_patched(const StemModel *m, const float *input, int H, int W, float *logits, int P);
int bnn_stem_forward_patched_device(const StemModel *m, const float *d_input, int H, int W, float *d_logits,
                                    int P, void *stream);
/* stages as in bnn_forward_debug, named as in the reference's v2 forward:
 * stem.conv (float), stem.act, enc1.conv1.P, enc1.act1, ... (the v1 names
 * from enc1.conv2.P on), logits */
typedef void (*bnn_stem_stage_cb)(void *ctx, const char *name, int dtype, int n, int c,
                                  int h, int w, const void *data);
int bnn_stem_forward_debug(const StemModel *m, const float *input, int N, int H, int W,
                           float *logits, bnn_stem_stage_cb cb, void *ctx);

#ifdef __cplusplus
}
#endif
#endif
