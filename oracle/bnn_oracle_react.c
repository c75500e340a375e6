/* bnn_oracle_react.c - CPU restatement of the reference v3 (ReActNet,
 * real-highway) forward.  TEST INFRASTRUCTURE ONLY: the checker the HIP v3
 * engine is compared against; nothing in the product links it.
 *
 * Semantics follow the reference C engine as its Makefile.react builds it
 * (gcc -O3 -march=native on an FMA host, so a*b + c contracts to one fused
 * multiply-add, written here as fmaf; the file is compiled with
 * -ffp-contract=off so that every other operation rounds on its own):
 *   blob parse ............ csrc/bnn_model_react.c:44-135
 *   forward ............... csrc/bnn_model_react.c:140-274, 395-438
 *                           (enc1 and dec1 run in row strips there; strips of
 *                           an even number of rows with a 2-row halo give the
 *                           whole-image values, so this runs the whole image)
 *   patch-wise forward .... csrc/bnn_model_react.c:454-476
 *   proj (1x1, real W) .... csrc/bnn_realin_blk.h:39-83, bnn_react_ops.c:117-133
 *   enc1 3x3 real conv .... csrc/bnn_realin_blk.h:85-152 (Cout % 8 == 0),
 *                           else the v1 conv_realin order (orc_conv_real)
 *   epilogues ............. csrc/bnn_react_epi.c:34-77
 *   tap ................... csrc/bnn_react_ops.c:75-85
 *   real / P max-pool ..... csrc/bnn_react_opt.c:47-83
 *   up + concat ........... csrc/bnn_model_react.c:280-298
 *   head .................. csrc/bnn_react_opt.c:23-44 (x86: the scalar loop)
 *   binary conv P ......... orc_bconv (the integers every reference bconv
 *                           kernel gives, int16 storage included)
 */
#include "bnn_oracle.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define TAG_BIN 1
#define TAG_REAL 2
#define TAG_HEAD 4
#define TAG_PROJ 5
#define TAG_EPI 6
#define TAG_TAP 7

/* ------------------------------------------------------------------ blob */
typedef struct {
    const uint8_t *p;
    size_t n, o;
    char *err;
    int errlen, bad;
} rreader;

static void rfail(rreader *r, const char *fmt, ...) {
    if (r->bad) return;
    r->bad = 1;
    if (r->err && r->errlen > 0) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(r->err, (size_t)r->errlen, fmt, ap);
        va_end(ap);
    }
}

static int32_t ri32(rreader *r) {
    int32_t v = 0;
    if (r->bad) return 0;
    if (r->n - r->o < 4) { rfail(r, "short read"); return 0; }
    memcpy(&v, r->p + r->o, 4);
    r->o += 4;
    return v;
}

/* n elements of elem bytes, checked against what is left before allocating */
static void *rtake(rreader *r, long long n, size_t elem) {
    if (r->bad) return NULL;
    if (n < 0) { rfail(r, "negative record dimension"); return NULL; }
    if ((long double)n * elem > (long double)(r->n - r->o)) { rfail(r, "short read"); return NULL; }
    size_t b = (size_t)n * elem;
    void *d = malloc(b ? b : 1);
    if (!d) { rfail(r, "out of memory"); return NULL; }
    memcpy(d, r->p + r->o, b);
    r->o += b;
    return d;
}

static void rconv(rreader *r, orc_conv *c) {
    memset(c, 0, sizeof *c);
    c->tag = ri32(r);
    c->cout = ri32(r); c->cin = ri32(r); c->kh = ri32(r); c->kw = ri32(r);
    c->pad = ri32(r); c->stride = ri32(r);
    if (r->bad) return;
    if (c->tag == TAG_BIN) {
        c->nwords = ri32(r);
        c->bits = rtake(r, (long long)c->cout * c->nwords, 8);
    } else if (c->tag == TAG_REAL) {
        if (c->cout < 0 || c->cin < 0 || c->kh < 0 || c->kw < 0) { rfail(r, "negative record dimension"); return; }
        c->wsign = rtake(r, (long long)c->cout * c->cin * c->kh * c->kw, 1);
        c->alpha = rtake(r, c->cout, 4);
    } else {
        rfail(r, "bad conv tag %d", c->tag);
    }
}

static void rproj(rreader *r, orr_proj_rec *p) {
    memset(p, 0, sizeof *p);
    int tag = ri32(r);
    if (!r->bad && tag != TAG_PROJ) { rfail(r, "bad proj tag %d", tag); return; }
    p->cout = ri32(r); p->cin = ri32(r);
    if (!r->bad && (p->cout < 0 || p->cin < 0)) { rfail(r, "negative record dimension"); return; }
    p->W = rtake(r, (long long)p->cout * p->cin, 4);
}

static void repi(rreader *r, orr_epi_rec *e) {
    memset(e, 0, sizeof *e);
    int tag = ri32(r);
    if (!r->bad && tag != TAG_EPI) { rfail(r, "bad epi tag %d", tag); return; }
    e->kind = ri32(r); e->c = ri32(r);
    e->A = rtake(r, e->c, 4); e->B = rtake(r, e->c, 4);
    e->move1 = rtake(r, e->c, 4); e->prelu_w = rtake(r, e->c, 4);
}

static void rtap(rreader *r, orr_tap_rec *t) {
    memset(t, 0, sizeof *t);
    int tag = ri32(r);
    if (!r->bad && tag != TAG_TAP) { rfail(r, "bad tap tag %d", tag); return; }
    t->c = ri32(r);
    t->rsign = rtake(r, t->c, 4);
}

static void rcheck(rreader *r, int ok, const char *what) {
    if (!ok) rfail(r, "blob layout mismatch: %s", what);
}

/* one block and the C loader's structural checks (csrc/bnn_model_react.c:86-106) */
static void rblock(rreader *r, orr_block *b, int is_down, int input_real) {
    memset(b, 0, sizeof *b);
    b->is_down = is_down; b->input_real = input_real;
    if (!input_real) rtap(r, &b->tap1);
    rconv(r, &b->c1); rproj(r, &b->p1); repi(r, &b->e1);
    rtap(r, &b->tap2); rconv(r, &b->c2); repi(r, &b->ea);
    if (is_down) repi(r, &b->eb);
    if (r->bad) return;
    rcheck(r, b->c1.tag == (input_real ? TAG_REAL : TAG_BIN), "conv1 tag");
    rcheck(r, b->c2.tag == TAG_BIN, "conv2 tag");
    rcheck(r, b->p1.cin == b->c1.cin && b->p1.cout == b->c1.cout, "proj1 dims");
    rcheck(r, input_real || b->tap1.c == b->c1.cin, "tap1 channels");
    rcheck(r, b->tap2.c == b->c2.cin, "tap2 channels");
    rcheck(r, b->e1.c == b->c1.cout && b->e1.kind == (input_real ? 1 : 0), "epi1");
    rcheck(r, b->ea.c == b->c2.cout && b->ea.kind == 0, "epi_a");
    rcheck(r, !is_down || (b->eb.c == b->c2.cout && b->eb.kind == 0), "epi_b");
}

static void free_epi(orr_epi_rec *e) { free(e->A); free(e->B); free(e->move1); free(e->prelu_w); }
static void free_cv(orc_conv *c) { free(c->bits); free(c->wsign); free(c->alpha); }
static void free_block(orr_block *b) {
    free(b->tap1.rsign); free(b->tap2.rsign);
    free_cv(&b->c1); free_cv(&b->c2); free(b->p1.W);
    free_epi(&b->e1); free_epi(&b->ea); free_epi(&b->eb);
}

void orr_free(orr_model *m) {
    if (!m) return;
    for (int i = 0; i < 4; ++i) { free_block(&m->enc[i]); free_block(&m->dec[i]); }
    free_block(&m->bott);
    free(m->head_w); free(m->head_b);
    free(m);
}

int orr_parse(const uint8_t *buf, size_t len, orr_model **out, char *err, int errlen) {
    rreader r = {buf, len, 0, err, errlen, 0};
    *out = NULL;
    if (len < 4 || memcmp(buf, "BNNC", 4) != 0) { rfail(&r, len < 4 ? "short read" : "bad magic"); return 1; }
    r.o = 4;
    orr_model *m = calloc(1, sizeof *m);
    if (!m) { rfail(&r, "out of memory"); return 1; }
    m->version = ri32(&r);
    if (!r.bad && m->version != 3) rfail(&r, "blob version %d, this engine reads v3 (ReActNet)", m->version);
    m->base = ri32(&r); m->n_bands = ri32(&r); m->n_classes = ri32(&r); m->upsampler = ri32(&r);
    if (!r.bad && m->upsampler != 0) rfail(&r, "only nearest upsampler supported");
    for (int i = 0; i < 4; ++i) rblock(&r, &m->enc[i], 1, i == 0);
    rblock(&r, &m->bott, 0, 0);
    for (int i = 0; i < 4; ++i) rblock(&r, &m->dec[i], 0, 0);
    int tag = ri32(&r);
    if (!r.bad && tag != TAG_HEAD) rfail(&r, "bad head tag %d", tag);
    m->head_cout = ri32(&r); m->head_cin = ri32(&r);
    if (!r.bad && (m->head_cout < 0 || m->head_cin < 0)) rfail(&r, "negative record dimension");
    m->head_w = rtake(&r, (long long)m->head_cout * m->head_cin, 4);
    m->head_b = rtake(&r, m->head_cout, 4);
    if (!r.bad && r.o != r.n) rfail(&r, "trailing bytes in blob");
    if (r.bad) { orr_free(m); return 1; }
    *out = m;
    return 0;
}

/* -------------------------------------------------------------- kernels */
/* 1x1 real projection, no bias: per output one chain over ci from 0,
 * acc = fma(W, x, acc) from +0 (csrc/bnn_realin_blk.h:59-70; the scalar
 * pixel tail of :76-81 and react_proj_1x1 run the same chain) */
void orr_proj(const float *x, const float *Wm, float *out, int cin, int HW, int cout) {
    /* outputs in parallel; each is one thread's chain */
    #pragma omp parallel for collapse(2) schedule(static)
    for (int co = 0; co < cout; ++co)
        for (long p = 0; p < HW; ++p) {
            float acc = 0.0f;
            for (int ci = 0; ci < cin; ++ci)
                acc = fmaf(Wm[(size_t)co * cin + ci], x[(size_t)ci * HW + p], acc);
            out[(size_t)co * HW + p] = acc;
        }
}

/* 3x3 / pad 1 / stride 1 real-input conv with +-1 weights, the register-
 * blocked order (csrc/bnn_realin_blk.h:111-147): per output one chain,
 * input channels outermost, then the taps row-major; a tap outside the
 * image is skipped; finally alpha * acc. */
void orr_conv3(const float *x, const int8_t *wsign, const float *alpha, float *out,
               int cin, int H, int W, int cout) {
    /* outputs in parallel; each is one thread's chain */
    #pragma omp parallel for collapse(2) schedule(static)
    for (int co = 0; co < cout; ++co)
        for (int oy = 0; oy < H; ++oy)
            for (int ox = 0; ox < W; ++ox) {
                float acc = 0.0f;
                for (int ci = 0; ci < cin; ++ci)
                    for (int ky = 0; ky < 3; ++ky) {
                        const int iy = oy + ky - 1;
                        if (iy < 0 || iy >= H) continue;
                        for (int kx = 0; kx < 3; ++kx) {
                            const int ix = ox + kx - 1;
                            if (ix < 0 || ix >= W) continue;
                            acc = fmaf((float)wsign[((size_t)co * cin + ci) * 9 + ky * 3 + kx],
                                       x[((size_t)ci * H + iy) * W + ix], acc);
                        }
                    }
                out[((size_t)co * H + oy) * W + ox] = alpha[co] * acc;
            }
}

/* t = fma(A, acc, B + move1) + res; out = t >= 0 ? t : prelu_w * t
 * (csrc/bnn_react_epi.c:34-55, :57-77) */
static inline float epi1(float A, float acc, float Bm, float res, float w) {
    const float t = fmaf(A, acc, Bm) + res;
    return t >= 0.0f ? t : w * t;
}

void orr_epi_int(const int32_t *P, const float *res, float *out, int C, int HW,
                 const float *A, const float *B, const float *move1, const float *prelu_w) {
    for (int c = 0; c < C; ++c) {
        const float Bm = B[c] + move1[c];
        for (long p = 0; p < HW; ++p) {
            const size_t i = (size_t)c * HW + p;
            out[i] = epi1(A[c], (float)P[i], Bm, res[i], prelu_w[c]);
        }
    }
}

void orr_epi_real(const float *x, const float *res, float *out, int C, int HW,
                  const float *A, const float *B, const float *move1, const float *prelu_w) {
    for (int c = 0; c < C; ++c) {
        const float Bm = B[c] + move1[c];
        for (long p = 0; p < HW; ++p) {
            const size_t i = (size_t)c * HW + p;
            out[i] = epi1(A[c], x[i], Bm, res[i], prelu_w[c]);
        }
    }
}

/* the first epilogue form, which the forward does not call: t = A*acc + B +
 * res + move1 in that order, the first product and add fused
 * (csrc/bnn_react_ops.c:36-70); acc int32 (is_int) or float */
void orr_epi_plain(const void *acc, int is_int, const float *res, float *out, int C, int HW,
                   const float *A, const float *B, const float *move1, const float *prelu_w) {
    for (int c = 0; c < C; ++c)
        for (long p = 0; p < HW; ++p) {
            const size_t i = (size_t)c * HW + p;
            const float v = is_int ? (float)((const int32_t *)acc)[i] : ((const float *)acc)[i];
            const float t = (fmaf(A[c], v, B[c]) + res[i]) + move1[c];
            out[i] = t >= 0.0f ? t : prelu_w[c] * t;
        }
}

/* sign(x + rsign) as +-1, x + rsign == 0 -> -1 (csrc/bnn_react_ops.c:75-85) */
void orr_tap(const float *x, int8_t *out, int C, int HW, const float *rsign) {
    for (int c = 0; c < C; ++c)
        for (long p = 0; p < HW; ++p) {
            const size_t i = (size_t)c * HW + p;
            out[i] = (x[i] + rsign[c] > 0.0f) ? 1 : -1;
        }
}

/* 2x2 / stride 2 floor-mode max, first of equal values kept, reading
 * (0,0), (0,1), (1,0), (1,1) (csrc/bnn_react_opt.c:61-66) */
void orr_maxpool_real(const float *x, float *out, int C, int H, int W) {
    const int Ho = H / 2, Wo = W / 2;
    for (int c = 0; c < C; ++c)
        for (int oy = 0; oy < Ho; ++oy)
            for (int ox = 0; ox < Wo; ++ox) {
                const float *r0 = x + ((size_t)c * H + 2 * oy) * W + 2 * ox, *r1 = r0 + W;
                float m = r0[0];
                if (r0[1] > m) m = r0[1];
                if (r1[0] > m) m = r1[0];
                if (r1[1] > m) m = r1[1];
                out[((size_t)c * Ho + oy) * Wo + ox] = m;
            }
}

/* [skip; nearest-2x up of x] on channels, the up part placed at the F.pad
 * before-offset, everything it does not cover 0.0 (csrc/bnn_model_react.c:280-298) */
void orr_up_cat(const float *skip, int sC, int sH, int sW, const float *x, int xC, int hH, int hW,
                float *out) {
    memcpy(out, skip, (size_t)sC * sH * sW * sizeof(float));
    memset(out + (size_t)sC * sH * sW, 0, (size_t)xC * sH * sW * sizeof(float));
    const int upH = 2 * hH, upW = 2 * hW, dh = sH - upH, dw = sW - upW;
    const int oh = dh > 0 ? dh / 2 : 0, ow = dw > 0 ? dw / 2 : 0;
    const int cH = upH < sH ? upH : sH, cW = upW < sW ? upW : sW;
    for (int c = 0; c < xC; ++c)
        for (int y = 0; y < cH; ++y)
            for (int xx = 0; xx < cW; ++xx)
                out[((size_t)(sC + c) * sH + oh + y) * sW + ow + xx] = x[((size_t)c * hH + y / 2) * hW + xx / 2];
}

/* bias, then channels in order, one fused step each (csrc/bnn_react_opt.c:33-41) */
void orr_head(const float *a, const float *Wm, const float *bias, float *out, int cin, int HW, int cout) {
    for (int o = 0; o < cout; ++o)
        for (long p = 0; p < HW; ++p) {
            float acc = bias[o];
            for (int c = 0; c < cin; ++c) acc = fmaf(Wm[(size_t)o * cin + c], a[(size_t)c * HW + p], acc);
            out[(size_t)o * HW + p] = acc;
        }
}

/* -------------------------------------------------------------- forward */
static int bin3(const orc_conv *c) {
    return c->tag == TAG_BIN && c->kh == 3 && c->kw == 3 && c->pad == 1 && c->stride == 1 &&
           c->nwords == (c->cin * 9 + 63) / 64;
}

/* The widths must chain as the forward uses them; the reference trusts the
 * blob here, this checker refuses instead. */
static int model_ok(const orr_model *m, int H, int W) {
    if (H < 16 || W < 16) return 0;
    int prev = m->n_bands;
    int skipC[4];
    for (int i = 0; i < 4; ++i) {
        const orr_block *b = &m->enc[i];
        if (b->c1.cin != prev || b->c2.cin != b->c1.cout || b->c2.cout != b->c1.cout) return 0;
        if (i == 0 ? (b->c1.kh != b->c1.kw || b->c1.stride != 1 || 2 * b->c1.pad != b->c1.kh - 1)
                   : !bin3(&b->c1))
            return 0;
        if (!bin3(&b->c2)) return 0;
        skipC[i] = b->c2.cout;
        prev = b->c2.cout;
    }
    const orr_block *bt = &m->bott;
    if (bt->c1.cin != prev || !bin3(&bt->c1) || !bin3(&bt->c2) || bt->c2.cin != bt->c1.cout ||
        bt->c2.cout != bt->c1.cout)
        return 0;
    prev = bt->c2.cout;
    for (int i = 0; i < 4; ++i) {
        const orr_block *b = &m->dec[i];
        if (b->c1.cin != skipC[3 - i] + prev || !bin3(&b->c1) || !bin3(&b->c2) ||
            b->c2.cin != b->c1.cout || b->c2.cout != b->c1.cout)
            return 0;
        prev = b->c2.cout;
    }
    return m->head_cin == prev && m->head_cout == m->n_classes;
}

static void emit(orc_stage_cb cb, void *ctx, const char *name, int dt, int c, int h, int w, const void *d) {
    if (cb) cb(ctx, name, dt, c, h, w, d);
}

static void *xal(size_t n) {
    void *p = malloc(n ? n : 1);
    if (!p) { fprintf(stderr, "oracle: out of memory\n"); abort(); }
    return p;
}

static int32_t *bconv_of(const orc_conv *c, const int8_t *a, int H, int W) {
    int32_t *P = xal((size_t)c->cout * H * W * 4);
    orc_bconv(a, c->bits, P, c->cin, H, W, c->cout, 3, 3, 1, 1);
    return P;
}

/* unit 1 of a binary-input block: h1 = epi1(P(tap1(x)), proj(x)) */
static float *unit1_bin(const orr_block *b, const float *x, int H, int W, const char *nm,
                        orc_stage_cb cb, void *ctx) {
    char s[48];
    const int HW = H * W, co = b->c1.cout;
    float *res = xal((size_t)co * HW * 4);
    orr_proj(x, b->p1.W, res, b->p1.cin, HW, co);
    snprintf(s, sizeof s, "%s.u1.proj", nm); emit(cb, ctx, s, 2, co, H, W, res);
    int8_t *a = xal((size_t)b->c1.cin * HW);
    orr_tap(x, a, b->c1.cin, HW, b->tap1.rsign);
    snprintf(s, sizeof s, "%s.u1.tap", nm); emit(cb, ctx, s, 0, b->c1.cin, H, W, a);
    int32_t *P = bconv_of(&b->c1, a, H, W);
    free(a);
    snprintf(s, sizeof s, "%s.u1.P", nm); emit(cb, ctx, s, 1, co, H, W, P);
    orr_epi_int(P, res, res, co, HW, b->e1.A, b->e1.B, b->e1.move1, b->e1.prelu_w);
    free(P);
    snprintf(s, sizeof s, "%s.h1", nm); emit(cb, ctx, s, 2, co, H, W, res);
    return res;
}

/* tap2 and conv2 of any block: P2 */
static int32_t *unit2_P(const orr_block *b, const float *h1, int H, int W, const char *nm,
                        orc_stage_cb cb, void *ctx) {
    char s[48];
    int8_t *a = xal((size_t)b->c2.cin * H * W);
    orr_tap(h1, a, b->c2.cin, H * W, b->tap2.rsign);
    snprintf(s, sizeof s, "%s.u2.tap", nm); emit(cb, ctx, s, 0, b->c2.cin, H, W, a);
    int32_t *P = bconv_of(&b->c2, a, H, W);
    free(a);
    snprintf(s, sizeof s, "%s.u2.P", nm); emit(cb, ctx, s, 1, b->c2.cout, H, W, P);
    return P;
}

int orr_forward(const orr_model *m, const float *in, int H, int W, float *logits, orc_stage_cb cb, void *ctx) {
    if (!model_ok(m, H, W)) return 1;
    static const char *EN[4] = {"enc1", "enc2", "enc3", "enc4"};
    static const char *DN[4] = {"dec4", "dec3", "dec2", "dec1"};
    char s[48];
    float *skip[4];
    int sC[4], sH[4], sW[4];
    const float *x = in;
    float *xo = NULL;
    int h = H, w = W;
    for (int i = 0; i < 4; ++i) {
        const orr_block *b = &m->enc[i];
        const int co = b->c2.cout, HW = h * w;
        float *h1;
        if (b->input_real) {
            const orc_conv *c = &b->c1;
            float *res = xal((size_t)c->cout * HW * 4), *cv = xal((size_t)c->cout * HW * 4);
            orr_proj(x, b->p1.W, res, b->p1.cin, HW, c->cout);
            emit(cb, ctx, "enc1.u1.proj", 2, c->cout, h, w, res);
            if (c->kh == 3 && c->kw == 3 && c->pad == 1 && c->stride == 1 && c->cout % 8 == 0)
                orr_conv3(x, c->wsign, c->alpha, cv, c->cin, h, w, c->cout);
            else
                orc_conv_real(x, c->wsign, c->alpha, cv, c->cin, h, w, c->cout, c->kh, c->kw, c->pad, c->stride);
            emit(cb, ctx, "enc1.u1.conv", 2, c->cout, h, w, cv);
            orr_epi_real(cv, res, res, c->cout, HW, b->e1.A, b->e1.B, b->e1.move1, b->e1.prelu_w);
            free(cv);
            h1 = res;
            emit(cb, ctx, "enc1.h1", 2, c->cout, h, w, h1);
        } else {
            h1 = unit1_bin(b, x, h, w, EN[i], cb, ctx);
        }
        int32_t *P2 = unit2_P(b, h1, h, w, EN[i], cb, ctx);
        float *sk = xal((size_t)co * HW * 4);
        orr_epi_int(P2, h1, sk, co, HW, b->ea.A, b->ea.B, b->ea.move1, b->ea.prelu_w);
        snprintf(s, sizeof s, "%s.skip", EN[i]); emit(cb, ctx, s, 2, co, h, w, sk);
        const int hh = h / 2, wh = w / 2;
        int32_t *Pd = xal((size_t)co * hh * wh * 4);
        orc_maxpool(P2, Pd, co, h, w, 2, 2);
        free(P2);
        snprintf(s, sizeof s, "%s.pool.P", EN[i]); emit(cb, ctx, s, 1, co, hh, wh, Pd);
        float *dn = xal((size_t)co * hh * wh * 4);
        orr_maxpool_real(h1, dn, co, h, w);
        free(h1);
        snprintf(s, sizeof s, "%s.pool.h", EN[i]); emit(cb, ctx, s, 2, co, hh, wh, dn);
        orr_epi_int(Pd, dn, dn, co, hh * wh, b->eb.A, b->eb.B, b->eb.move1, b->eb.prelu_w);
        free(Pd);
        snprintf(s, sizeof s, "%s.down", EN[i]); emit(cb, ctx, s, 2, co, hh, wh, dn);
        skip[i] = sk; sC[i] = co; sH[i] = h; sW[i] = w;
        free(xo);
        xo = dn; x = dn; h = hh; w = wh;
    }
    {
        const orr_block *b = &m->bott;
        float *h1 = unit1_bin(b, x, h, w, "bott", cb, ctx);
        int32_t *P2 = unit2_P(b, h1, h, w, "bott", cb, ctx);
        orr_epi_int(P2, h1, h1, b->c2.cout, h * w, b->ea.A, b->ea.B, b->ea.move1, b->ea.prelu_w);
        free(P2);
        emit(cb, ctx, "bott.h2", 2, b->c2.cout, h, w, h1);
        free(xo);
        xo = h1; x = h1;
    }
    int xc = m->bott.c2.cout;
    for (int i = 0; i < 4; ++i) {
        const orr_block *b = &m->dec[i];
        const int si = 3 - i, H2 = sH[si], W2 = sW[si], HW = H2 * W2;
        float *cat = xal((size_t)(sC[si] + xc) * HW * 4);
        orr_up_cat(skip[si], sC[si], H2, W2, x, xc, h, w, cat);
        free(skip[si]);
        snprintf(s, sizeof s, "%s.cat", DN[i]); emit(cb, ctx, s, 2, sC[si] + xc, H2, W2, cat);
        float *h1 = unit1_bin(b, cat, H2, W2, DN[i], cb, ctx);
        free(cat);
        int32_t *P2 = unit2_P(b, h1, H2, W2, DN[i], cb, ctx);
        orr_epi_int(P2, h1, h1, b->c2.cout, HW, b->ea.A, b->ea.B, b->ea.move1, b->ea.prelu_w);
        free(P2);
        snprintf(s, sizeof s, "%s.h2", DN[i]); emit(cb, ctx, s, 2, b->c2.cout, H2, W2, h1);
        free(xo);
        xo = h1; x = h1; h = H2; w = W2; xc = b->c2.cout;
    }
    orr_head(x, m->head_w, m->head_b, logits, m->head_cin, h * w, m->head_cout);
    emit(cb, ctx, "logits", 2, m->head_cout, h, w, logits);
    free(xo);
    return 0;
}

/* independent P x P patches, edge patches zero past the image, stitched
 * (csrc/bnn_model_react.c:454-476) */
int orr_forward_patched(const orr_model *m, const float *in, int H, int W, float *logits, int P) {
    if (P <= 0 || P % 16 || !model_ok(m, P, P)) return 1;
    const int nb = m->n_bands, nc = m->n_classes;
    float *pin = xal((size_t)nb * P * P * 4), *pout = xal((size_t)nc * P * P * 4);
    for (int py = 0; py < H; py += P) {
        const int ph = py + P < H ? P : H - py;
        for (int px = 0; px < W; px += P) {
            const int pw = px + P < W ? P : W - px;
            memset(pin, 0, (size_t)nb * P * P * 4);
            for (int b = 0; b < nb; ++b)
                for (int y = 0; y < ph; ++y)
                    memcpy(pin + ((size_t)b * P + y) * P, in + ((size_t)b * H + py + y) * W + px, (size_t)pw * 4);
            orr_forward(m, pin, P, P, pout, NULL, NULL);
            for (int c = 0; c < nc; ++c)
                for (int y = 0; y < ph; ++y)
                    memcpy(logits + ((size_t)c * H + py + y) * W + px, pout + ((size_t)c * P + y) * P, (size_t)pw * 4);
        }
    }
    free(pin); free(pout);
    return 0;
}

/* N patches, one per OpenMP thread */
int orr_forward_batch_par(const orr_model *m, const float *in, int N, int H, int W, float *logits) {
    if (!model_ok(m, H, W)) return 1;
    const size_t si = (size_t)m->n_bands * H * W, so = (size_t)m->n_classes * H * W;
    int bad = 0;
#pragma omp parallel for schedule(dynamic, 1) reduction(| : bad)
    for (int n = 0; n < N; ++n) bad |= orr_forward(m, in + n * si, H, W, logits + n * so, NULL, NULL);
    return bad;
}
