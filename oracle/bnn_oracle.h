/* bnn_oracle.h - CPU restatement of the reference v1 Bi-Real UNet forward.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the HIP engine is
 * compared against (and the "port" CPU baseline in bench.py).  Nothing in the
 * product links it, loads it or falls back to it.
 *
 * Semantics follow the reference C engine (csrc/ of Sboyle132/BNNs_to_C):
 *   blob parse ................ csrc/bnn_model.c:27-96 (+ python/bnn2c/blob.py:159-200)
 *   forward stage order ....... csrc/bnn_model.c:150-253
 *   binary conv P ............. csrc/bnn_conv.c:23-36, 50-223
 *   real-input first conv ..... csrc/bnn_conv_realin.c:66-116, 140-172
 *   folds ..................... csrc/bnn_fold.c:37-77
 *   max-pool on P ............. csrc/bnn_maxpool.c:28-48
 *   nearest up + concat ....... csrc/bnn_model.c:130-148
 *   head ...................... csrc/bnn_head.c:21-34
 * Float evaluation order is the reference's as built by its Makefile
 * (gcc -O3 -march=native on an FMA host): in-order sums, and a fused
 * multiply-add only in the real fold's z = A*x + B.
 */
#ifndef BNN_ORACLE_H
#define BNN_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int tag;                  /* 1 binary (kidx-packed bits), 2 real (wsign + alpha) */
    int cout, cin, kh, kw, pad, stride, nwords;
    uint64_t *bits;
    int8_t *wsign;
    float *alpha;
} orc_conv;

typedef struct {
    int kind, c;              /* 0 integer rule on P, 1 real fold */
    int32_t *type, *t, *lo, *hi;
    float *A, *B, *slope, *rsign;
} orc_act;

typedef struct {
    int version, base, n_bands, n_classes, upsampler;
    /* v2 (csrc/bnn_model_stem.h:38-56): a real-input 1x1 binary-weight stem
     * and real fold before a uniformly binary encoder (enc1.conv1 binary) */
    int has_stem, n_stem_layers;
    orc_conv stem_c;
    orc_act stem_a;
    orc_conv enc_c1[4], enc_c2[4];
    orc_act enc_a1[4], enc_skip[4], enc_down[4];
    orc_conv bott_c1, bott_c2;
    orc_act bott_a1, bott_a2;
    orc_conv dec_c1[4], dec_c2[4];           /* index 0..3 = dec4..dec1 */
    orc_act dec_a1[4], dec_a2[4];
    int head_cout, head_cin;
    float *head_w, *head_b;
} orc_model;

/* ---- blob ---- */
int  orc_parse(const uint8_t *buf, size_t len, int strict, orc_model **out,
               char *err, int errlen);
void orc_free(orc_model *m);

/* ---- forward ----
 * Stage callback: dtype 0 = int8 +-1, 1 = int32 accumulator P, 2 = float32.
 * Names: enc1.conv1, enc1.act1 (v1) or stem.conv, stem.act, enc1.conv1.P,
 * enc1.act1 (v2), encK.conv1.P (K>1), encK.act1, encK.conv2.P,
 * encK.act2_skip, encK.pool.P, encK.act2_down, bott.conv{1,2}.P, bott.act{1,2},
 * decK.upcat, decK.conv{1,2}.P, decK.act{1,2}, logits. */
typedef void (*orc_stage_cb)(void *ctx, const char *name, int dtype,
                             int c, int h, int w, const void *data);
int orc_forward(const orc_model *m, const float *in, int H, int W,
                float *logits, orc_stage_cb cb, void *ctx);
/* N patches in sequence through orc_forward (threads only inside bconv) */
int orc_forward_batch(const orc_model *m, const float *in, int N, int H, int W,
                      float *logits);
/* N patches, one patch per OpenMP thread (a faster checker, same results) */
int orc_forward_batch_par(const orc_model *m, const float *in, int N, int H,
                          int W, float *logits);

/* ---- kernels (batch 1, row-major, same argument meaning as the reference) */
void orc_pack_kidx(const int8_t *wsign, uint64_t *bits, int cout, int cin,
                   int kh, int kw);
void orc_bconv_naive(const int8_t *a, const int8_t *wsign, int32_t *P, int cin,
                     int H, int W, int cout, int kh, int kw, int pad, int stride);
void orc_bconv_dense(const int8_t *a, const uint64_t *bits, int32_t *P, int cin,
                     int H, int W, int cout, int kh, int kw, int pad, int stride);
void orc_bconv_chan(const int8_t *a, const uint64_t *bits, int32_t *P, int cin,
                    int H, int W, int cout, int kh, int kw, int pad, int stride);
void orc_bconv(const int8_t *a, const uint64_t *bits, int32_t *P, int cin,
               int H, int W, int cout, int kh, int kw, int pad, int stride);
void orc_conv_real(const float *x, const int8_t *wsign, const float *alpha,
                   float *out, int cin, int H, int W, int cout, int kh, int kw,
                   int pad, int stride);
void orc_fold_int(const int32_t *P, int8_t *out, int C, int H, int W,
                  const int32_t *type, const int32_t *t, const int32_t *lo,
                  const int32_t *hi);
void orc_fold_real(const float *x, int8_t *out, int C, int H, int W,
                   const float *A, const float *B, const float *slope,
                   const float *rsign);
void orc_maxpool(const int32_t *P, int32_t *out, int C, int H, int W, int k,
                 int stride);
void orc_head(const float *a, const float *Wt, const float *bias, float *logits,
              int cin, int H, int W, int cout);
void orc_up_cat(const int8_t *skip, int sC, int sH, int sW, const int8_t *x,
                int xC, int hH, int hW, int8_t *out);

/* ---- v3 (ReActNet real highway; bnn_oracle_react.c) ----
 * Records of csrc/bnn_model_react.h:57-88; dec[0..3] = dec4..dec1. */
typedef struct { int c; float *rsign; } orr_tap_rec;
typedef struct { int cout, cin; float *W; } orr_proj_rec;
typedef struct { int kind, c; float *A, *B, *move1, *prelu_w; } orr_epi_rec;
typedef struct {
    int is_down, input_real;
    orr_tap_rec tap1, tap2;
    orc_conv c1, c2;
    orr_proj_rec p1;
    orr_epi_rec e1, ea, eb;       /* ea: skip (down) or epi2 (plain); eb: pooled down */
} orr_block;
typedef struct {
    int version, base, n_bands, n_classes, upsampler;
    orr_block enc[4], bott, dec[4];
    int head_cout, head_cin;
    float *head_w, *head_b;
} orr_model;

int  orr_parse(const uint8_t *buf, size_t len, orr_model **out, char *err, int errlen);
void orr_free(orr_model *m);
/* Stages (dtype as orc_forward): enc1.u1.proj, enc1.u1.conv, enc1.h1;
 * X.u1.proj, X.u1.tap, X.u1.P, X.h1 (X = enc2..4, bott, dec4..1);
 * X.u2.tap, X.u2.P; encK.skip, encK.pool.P, encK.pool.h, encK.down;
 * bott.h2, decK.cat, decK.h2; logits. */
int  orr_forward(const orr_model *m, const float *in, int H, int W, float *logits,
                 orc_stage_cb cb, void *ctx);
int  orr_forward_patched(const orr_model *m, const float *in, int H, int W, float *logits, int P);
int  orr_forward_batch_par(const orr_model *m, const float *in, int N, int H, int W, float *logits);
void orr_proj(const float *x, const float *Wm, float *out, int cin, int HW, int cout);
void orr_conv3(const float *x, const int8_t *wsign, const float *alpha, float *out,
               int cin, int H, int W, int cout);
void orr_epi_int(const int32_t *P, const float *res, float *out, int C, int HW,
                 const float *A, const float *B, const float *move1, const float *prelu_w);
void orr_epi_real(const float *x, const float *res, float *out, int C, int HW,
                  const float *A, const float *B, const float *move1, const float *prelu_w);
void orr_epi_plain(const void *acc, int is_int, const float *res, float *out, int C, int HW,
                   const float *A, const float *B, const float *move1, const float *prelu_w);
void orr_tap(const float *x, int8_t *out, int C, int HW, const float *rsign);
void orr_maxpool_real(const float *x, float *out, int C, int H, int W);
void orr_up_cat(const float *skip, int sC, int sH, int sW, const float *x, int xC, int hH, int hW,
                float *out);
void orr_head(const float *a, const float *Wm, const float *bias, float *out, int cin, int HW, int cout);

#ifdef __cplusplus
}
#endif
#endif
