/* bnn_model.h - C ABI of libbnn_hip.so, the MI355X (gfx950) engine for the
 * v1 nearest-upsampler Bi-Real binary UNet.
 *
 * Drop-in for the reference's csrc/bnn_model.h: the same record types, the
 * same Model field order, and the same load / forward / free and kernel
 * entry points with the same argument meaning.  Every entry point runs on
 * the GPU; host pointers in, host pointers out, synchronous on return,
 * unless the name says _device.  The reference-named entry points keep the
 * reference's error behaviour (message on stderr, exit(1)); the bnn_*_status
 * extensions return an error code instead and leave the text in
 * bnn_last_error().
 */
#ifndef BNN_MODEL_H
#define BNN_MODEL_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- kernels: csrc/bnn_model.h:7-23 (+ csrc/bnn_conv.c:50,80) ----
 * Batch 1, contiguous row-major, exactly the reference's layouts:
 *   a [Cin,H,W] int8 +-1;  packed_w [Cout][ceil(Cin*kh*kw/64)] kidx-order
 *   sign bits;  P [Cout,Hout,Wout] int32;  x [Cin,H,W] float. */
void bconv_xnor(const int8_t *a, const uint64_t *packed_w, int32_t *P,
                int Cin, int H, int W, int Cout, int kh, int kw, int pad, int stride);
void bconv_xnor_packed(const int8_t *a, const uint64_t *packed_w, int32_t *P,
                int Cin, int H, int W, int Cout, int kh, int kw, int pad, int stride);
void bconv_dispatch(const int8_t *a, const uint64_t *packed_w, int32_t *P,
                int Cin, int H, int W, int Cout, int kh, int kw, int pad, int stride);
/* csrc/bnn_conv.c:50: the +-1 triple loop on int8 weights (a == 0 counts 0) */
void bconv_naive_int(const int8_t *a, const int8_t *wsign, int32_t *P,
                     int Cin, int H, int W, int Cout, int kh, int kw, int pad, int stride);
/* csrc/bnn_conv.c:80: host-side bit packing, no GPU involved */
void pack_weights(const int8_t *wsign, uint64_t *packed, int Cout, int Cin, int kh, int kw);
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

/* ---- parsed blob records: csrc/bnn_model.h:25-55 ---- */
typedef struct {
    int tag;                 /* 1 = binary (packed), 2 = real (wsign+alpha) */
    int Cout, Cin, kh, kw, pad, stride, nwords;
    uint64_t *packed;        /* binary conv */
    int8_t *wsign;           /* real conv */
    float *alpha;            /* real conv */
} Conv;

typedef struct {
    int kind;                /* 0 = integer-P fold, 1 = real fold */
    int C;
    int32_t *type, *t, *lo, *hi;     /* int fold */
    float *A, *B, *slope, *rsign;    /* real fold */
} Act;

struct BnnDevice;            /* GPU-resident weights, workspace and stream */

typedef struct {
    int version, base_channels, n_bands, n_classes, upsampler;
    Conv enc_conv1[4], enc_conv2[4];
    Act  enc_act1[4], enc_act2_skip[4], enc_act2_down[4];
    Conv bott_conv1, bott_conv2;
    Act  bott_act1, bott_act2;
    Conv dec_conv1[4], dec_conv2[4];     /* index 0..3 == dec4..dec1 */
    Act  dec_act1[4], dec_act2[4];
    int head_Cout, head_Cin;
    float *head_W, *head_bias;
    struct BnnDevice *dev;   /* not in the reference; owned by the library */
} Model;

/* ---- csrc/bnn_model.h:57-60 ---- */
Model *bnn_load(const char *path);   /* never NULL: exits(1) on any error */
void bnn_free(Model *m);
/* input: [n_bands, H, W] float; logits: [n_classes, H, W] float (caller allocs) */
void bnn_forward(const Model *m, const float *input, int H, int W, float *logits);

/* ---- extensions (no counterpart in the reference) ---- */
#define BNN_OK 0
#define BNN_EBLOB 1      /* malformed or unsupported blob */
#define BNN_EARG 2       /* bad argument or shape */
#define BNN_EHIP 3       /* HIP runtime / device error */

const char *bnn_last_error(void);
/* parse + validate a blob on the host only (no GPU touched) */
int bnn_blob_check(const char *path);
int bnn_load_status(const char *path, Model **out);
/* N independent patches: input [N, n_bands, H, W] -> logits [N, n_classes, H, W]
 * (host pointers; the v1 forward applied to each patch, csrc/bnn_model.c:150-253) */
int bnn_forward_batch(const Model *m, const float *input, int N, int H, int W, float *logits);
/* same on device pointers, enqueued on `stream` (a hipStream_t; NULL is the
 * HIP default stream, as everywhere in HIP); returns once enqueued.  Calls
 * that share a model must be ordered by the caller: they share its workspace. */
int bnn_forward_device(const Model *m, const float *d_input, int N, int H, int W,
                       float *d_logits, void *stream);
void *bnn_stream(const Model *m);      /* the model's own hipStream_t (used by the host-pointer calls) */

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): bnn_forward_device without any allocation.  The
 * inter-layer tensors live in a fixed device array of
 * BNN_NOALLOC_SCRATCH_BYTES per GPU, held from the first bnn_load on that GPU
 * until the process ends; a call whose tensors do not fit returns BNN_EARG
 * (32x32 patches of the base-16 UNet: up to 1,980 per call).  It runs on
 * `stream` alone (no side streams) and calls no hipMalloc, hipFree or
 * allocating library routine.  Every call on one GPU shares that array, and
 * nothing in it needs to start at zero: calls that overlap on one GPU, even
 * on different models, race and must be ordered by the caller. */
#define BNN_NOALLOC_SCRATCH_BYTES (48u << 20)
int bnn_forward_device_noalloc(const Model *m, const float *d_input, int N, int H, int W,
                               float *d_logits, void *stream);

/* Scene inference by independent P x P patches, the tiling of the reference's
 * csrc/bnn_model_react.c:454-476 (bnn_forward_react_patched) applied to the v1
 * forward: patches start at multiples of P (a multiple of 16), an edge patch
 * is zero past the scene, each patch runs as its own P x P image and its
 * logits inside the scene are written to the map.
 * input [n_bands][H][W], logits [n_classes][H][W]; the cube must be < 2 GiB.
 * Host pointers: the cube crosses PCIe in strips, overlapped with compute. */
int bnn_forward_patched(const Model *m, const float *input, int H, int W, float *logits, int P);
/* same on device pointers, enqueued on `stream` (NULL = HIP default stream) */
int bnn_forward_patched_device(const Model *m, const float *d_input, int H, int W, float *d_logits, int P,
                               void *stream);

/* Debug forward: host pointers, then every stage of the chain is handed to
 * `cb` as a host array [N][c][h][w] (dtype 0 int8 +-1, 1 int32 P, 2 float),
 * named as in the reference forward: enc1.conv1, enc1.act1, encK.conv1.P,
 * encK.act1, encK.conv2.P, encK.act2_skip, encK.pool.P, encK.act2_down,
 * bott.conv{1,2}.P, bott.act{1,2}, decK.conv{1,2}.P, decK.act{1,2}, logits. */
typedef void (*bnn_stage_cb)(void *ctx, const char *name, int dtype, int n, int c,
                             int h, int w, const void *data);
int bnn_forward_debug(const Model *m, const float *input, int N, int H, int W,
                      float *logits, bnn_stage_cb cb, void *ctx);

/* No counterpart in the reference.  The certified first conv's record since
 * the previous call (or the load): the outputs it decided from its bounded
 * approximation plus the ones it recomputed in the reference's order
 * (*outputs), and the recomputed ones (*undecided).  Waits for all work on
 * the model's GPU, then resets both counts.  Both are 0 for a model whose
 * first conv runs in the reference's order (BNN_CERT=0, general signs). */
int bnn_cert_stats(const Model *m, unsigned long long *undecided, unsigned long long *outputs);

/* Per-op GPU timing of the device forward (hipEvents around every kernel). */
void bnn_prof_enable(int on);
int bnn_prof_count(void);
int bnn_prof_get(int i, char *label, int label_len, char *optype, int optype_len,
                 double *ms, double *work);

/* Isolated kernels on device pointers (benchmark configs 1 and 2); `stream`
 * is a hipStream_t, NULL = the HIP default stream.
 * act: [N][H][W][ceil(Cin/32)] uint32 channel-packed sign bits;
 * wt:  kidx-packed weights as in the blob, [Cout][ceil(Cin*9/64)] uint64 (host). */
typedef struct BnnConvLayer BnnConvLayer;
BnnConvLayer *bnn_layer_create(const uint64_t *packed_w, int Cin, int Cout,
                               const int32_t *type1, const int32_t *t1, const int32_t *lo1, const int32_t *hi1,
                               const int32_t *type2, const int32_t *t2, const int32_t *lo2, const int32_t *hi2);
void bnn_layer_free(BnnConvLayer *L);
/* 3x3 pad 1 stride 1 accumulator P [N][Cout][H][W] int32 */
int bnn_layer_P_device(const BnnConvLayer *L, const uint32_t *d_act, int N, int H, int W,
                       int32_t *d_P, void *stream);
/* conv + rule 1 -> skip bits [N][H][W][ceil(Cout/32)]; 2x2 max of P + rule 2
 * -> down bits [N][H/2][W/2][ceil(Cout/32)]; d_skip may be NULL */
int bnn_layer_fold_pool_device(const BnnConvLayer *L, const uint32_t *d_act, int N, int H, int W,
                               uint32_t *d_skip, uint32_t *d_down, void *stream);
/* pack int8 +-1 activations [N][C][H][W] (device) into [N][H][W][ceil(C/32)] */
int bnn_pack_act_device(const int8_t *d_a, uint32_t *d_out, int N, int C, int H, int W, void *stream);

/* The integer rule of csrc/bnn_fold.c:37-60 rewritten per channel as
 * bit = ((uint32)(P - lo) < wid) ^ inv, valid for |P| < 2^30 (host only). */
void bnn_fold_canon(const int32_t *type, const int32_t *t, const int32_t *lo, const int32_t *hi,
                    int C, int32_t *out_lo, uint32_t *out_wid, uint8_t *out_inv);

#ifdef __cplusplus
}
#endif
#endif
