/* bnn_model_react.h - C ABI of libbnn_hip.so for the v3 (ReActNet,
 * real-highway) model: blob version 3, a float highway between blocks,
 * binarising taps before each binary conv, 1x1 real projections and
 * BN + add + RPReLU epilogues.
 *
 * Drop-in for the reference's csrc/bnn_model_react.h: the same record types
 * (ConvR, EpiR, TapR, ProjR, BlockR), the same ModelR field order (plus a
 * trailing device pointer, as Model has in bnn_model.h), and
 * bnn_load_react / bnn_free_react / bnn_forward_react and its file and
 * patch-wise variants with the reference's argument meaning and error
 * behaviour (message on stderr, exit(1)).  The reference's v3 kernel entry
 * points are declared here too, with its batch-1 layouts; every one runs on
 * the GPU.  The same library serves bnn_model.h and bnn_model_stem.h; the
 * error codes, bnn_last_error() and the profiler are the ones declared in
 * bnn_model.h.
 */
#ifndef BNN_MODEL_REACT_H
#define BNN_MODEL_REACT_H
#include <stdint.h>
#include <stdio.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- kernels: csrc/bnn_model_react.h:9-53 ----
 * Batch 1, contiguous row-major [C,H,W], exactly the reference's layouts
 * (int16 P where the name says _i16). */
void bconv_dispatch(const int8_t *a, const uint64_t *packed_w, int32_t *P,
                    int Cin, int H, int W, int Cout, int kh, int kw, int pad, int stride);
void conv_realin_naive(const float *x, const int8_t *wsign, const float *alpha,
                       float *out, int Cin, int H, int W, int Cout,
                       int kh, int kw, int pad, int stride);
void maxpool_P(const int32_t *P, int32_t *Pout, int C, int H, int W, int k, int stride);
void head_1x1(const float *a, const float *W, const float *bias,
              float *logits, int Cin, int H, int W_, int Cout);
void react_epilogue_int(const int32_t *P, const float *res, float *out,
                        int C, int H, int W, const float *A, const float *B,
                        const float *move1, const float *prelu_w);
void react_epilogue_real(const float *cin, const float *res, float *out,
                         int C, int H, int W, const float *A, const float *B,
                         const float *move1, const float *prelu_w);
void head_1x1_v2(const float *a, const float *W, const float *bias,
                 float *logits, int Cin, int H, int W_, int Cout);
void maxpool_real_v2(const float *x, float *out, int C, int H, int W, int k, int stride);
void maxpool_P_v2(const int32_t *x, int32_t *out, int C, int H, int W, int k, int stride);
void react_epilogue_int_v2(const int32_t *P, const float *res, float *out,
                           int C, int H, int W, const float *A, const float *B,
                           const float *move1, const float *prelu_w);
void react_epilogue_real_v2(const float *cin, const float *res, float *out,
                            int C, int H, int W, const float *A, const float *B,
                            const float *move1, const float *prelu_w);
void react_tap(const float *x, int8_t *out, int C, int H, int W, const float *rsign);
void maxpool_real(const float *x, float *out, int C, int H, int W, int k, int stride);
void react_proj_1x1(const float *x, const float *Wm, float *out,
                    int Cin, int H, int W, int Cout);
void bconv_blk_b4p4(const int8_t *a, const uint64_t *packed_w, int32_t *P,
                    int Cin, int H, int W, int Cout, int kh, int kw, int pad, int stride);
void bconv_blk_b4p4_i16(const int8_t *a, const uint64_t *packed_w, int16_t *P,
                        int Cin, int H, int W, int Cout, int kh, int kw, int pad, int stride);
void react_epilogue_int_i16(const int16_t *P, const float *res, float *out,
                            int C, int H, int W, const float *A, const float *B,
                            const float *move1, const float *prelu_w);
void maxpool_P_i16(const int16_t *x, int16_t *out, int C, int H, int W, int k, int stride);
void react_proj_blk(const float *x, const float *Wm, float *out,
                    int Cin, int H, int W, int Cout);
void react_conv3_blk(const float *x, const int8_t *wsign, const float *alpha,
                     float *out, int Cin, int H, int W, int Cout);

/* ---- parsed blob records: csrc/bnn_model_react.h:56-88 ---- */
typedef struct {
    int tag;                 /* 1 = binary (packed), 2 = real (wsign+alpha) */
    int Cout, Cin, kh, kw, pad, stride, nwords;
    uint64_t *packed;
    int8_t *wsign;
    float *alpha;
} ConvR;

typedef struct { int kind, C; float *A, *B, *move1, *prelu_w; } EpiR;  /* kind 0=int 1=real */
typedef struct { int C; float *rsign; } TapR;                          /* C==0: absent (enc1) */
typedef struct { int Cout, Cin; float *W; } ProjR;                     /* real 1x1, no bias */

typedef struct {
    int is_down;             /* 1: DownBlock (fork), 0: PlainBlock */
    int input_real;          /* enc1 only: conv1 consumes raw spectra, no tap1 */
    TapR  tap1, tap2;
    ConvR conv1, conv2;
    ProjR proj1;
    EpiR  epi1;
    EpiR  epi_a;             /* down: skip epilogue ; plain: epi2 */
    EpiR  epi_b;             /* down: pooled-down epilogue ; plain: unused */
} BlockR;

struct BnnReactDevice;

typedef struct {
    int version, base_channels, n_bands, n_classes, upsampler;
    BlockR enc[4], bott, dec[4];     /* dec[0..3] == dec4..dec1 */
    int head_Cout, head_Cin;
    float *head_W, *head_bias;
    struct BnnReactDevice *dev;      /* not in the reference; owned by the library */
} ModelR;

/* ---- csrc/bnn_model_react.h:90-98 ---- */
ModelR *bnn_load_react(const char *path);      /* never NULL: exits(1) on any error */
void bnn_free_react(ModelR *m);
/* input: [n_bands,H,W] float; logits: [n_classes,H,W] float (caller allocs) */
void bnn_forward_react(const ModelR *m, const float *input, int H, int W, float *logits);
/* the [n_bands,H,W] f32 cube read from in_f */
void bnn_forward_react_file(const ModelR *m, FILE *in_f, int H, int W, float *logits);
/* patch-wise forward: independent PxP patches (edge patches zero past the image) */
void bnn_forward_react_patched(const ModelR *m, const float *input, int H, int W, float *logits, int P);
/* same, the cube read from a file one patch row at a time */
void bnn_forward_react_patched_file(const ModelR *m, FILE *f, int H, int W, float *logits, int P);

/* ---- extensions (no counterpart in the reference), the v3 twins of the
 * bnn_model.h extensions of the same names without "_react" ----
 * Return BNN_OK or an error code (text in bnn_last_error()). */
int bnn_react_blob_check(const char *path);
int bnn_react_load_status(const char *path, ModelR **out);
/* N patches [N][n_bands][H][W] -> logits [N][n_classes][H][W], host pointers */
int bnn_react_forward_batch(const ModelR *m, const float *input, int N, int H, int W, float *logits);
/* the same on device pointers, enqueued on stream (a hipStream_t; NULL = the
 * HIP default stream, as everywhere in HIP); returns once enqueued */
int bnn_react_forward_device(const ModelR *m, const float *d_input, int N, int H, int W,
                             float *d_logits, void *stream);
void *bnn_react_stream(const ModelR *m); /* the model's own hipStream_t (used by the host-pointer calls) */
int bnn_react_forward_patched(const ModelR *m, const float *input, int H, int W, float *logits, int P);
int bnn_react_forward_patched_device(const ModelR *m, const float *d_input, int H, int W, float *d_logits,
                                     int P, void *stream);
/* Every stage the GPU forward materialises, [N][C][H][W], dtype 0 = int8
 * +-1, 1 = int32 P, 2 = float32, named as the CPU checker names them:
 * enc1.u1.proj, enc1.u1.conv, enc1.h1; X.u1.proj, X.u1.tap, X.u1.P, X.h1
 * (X = enc2..4, bott, dec4..1); X.u2.tap, X.u2.P; encK.skip, encK.pool.P,
 * encK.down; bott.h2, decK.h2; logits. */
typedef void (*bnn_react_stage_cb)(void *ctx, const char *name, int dtype, int n, int c,
                                   int h, int w, const void *data);
int bnn_react_forward_debug(const ModelR *m, const float *input, int N, int H, int W,
                            float *logits, bnn_react_stage_cb cb, void *ctx);

#ifdef __cplusplus
}
#endif
#endif
