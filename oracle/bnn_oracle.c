/* bnn_oracle.c - CPU restatement of the reference v1 Bi-Real UNet forward.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP engine and the "port"
 * CPU baseline.  The product never links or calls this file.
 *
 * Build flags are pinned in oracle/Makefile: -O3 -mavx2 -mfma
 * -ffp-contract=off -fopenmp.  Contraction is off so every float operation
 * below is exactly the one written; the single fused multiply-add the
 * reference build emits (z = A*x + B in the real fold) is written as fmaf().
 */
#include "bnn_oracle.h"

#include <limits.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define TAG_BIN 1
#define TAG_REAL 2
#define TAG_ACT 3
#define TAG_HEAD 4

/* ------------------------------------------------------------------ blob */
/* Record layout: python/bnn2c/blob.py:67-114; order: blob.py:181-199 and
 * csrc/bnn_model.c:74-91; no trailing bytes: csrc/bnn_model.c:93. */
typedef struct {
    const uint8_t *p;
    size_t n, o;
    char *err;
    int errlen;
    int bad;
} reader;

static void fail(reader *r, const char *fmt, ...) {
    if (r->bad) return;
    r->bad = 1;
    if (r->err && r->errlen > 0) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(r->err, (size_t)r->errlen, fmt, ap);
        va_end(ap);
    }
}

static void *take(reader *r, size_t nbytes) {
    if (r->bad) return NULL;
    if (nbytes > r->n - r->o) { fail(r, "short read"); return NULL; }
    const uint8_t *src = r->p + r->o;
    r->o += nbytes;
    void *dst = malloc(nbytes ? nbytes : 1);
    if (!dst) { fail(r, "out of memory"); return NULL; }
    memcpy(dst, src, nbytes);
    return dst;
}

static int32_t take_i32(reader *r) {
    int32_t v = 0;
    if (r->bad) return 0;
    if (r->n - r->o < 4) { fail(r, "short read"); return 0; }
    memcpy(&v, r->p + r->o, 4);
    r->o += 4;
    return v;
}

/* element counts are checked against the bytes left before allocating */
static size_t count_or_fail(reader *r, long long a, long long b, long long c,
                            long long d, size_t elem) {
    if (a < 0 || b < 0 || c < 0 || d < 0) { fail(r, "negative record dimension"); return 0; }
    long double tot = (long double)a * b * c * d * elem;
    if (tot > (long double)(r->n - r->o)) { fail(r, "short read"); return 0; }
    return (size_t)(a * b * c * d);
}

static void parse_conv(reader *r, orc_conv *c) {
    memset(c, 0, sizeof *c);
    c->tag = take_i32(r);
    c->cout = take_i32(r); c->cin = take_i32(r);
    c->kh = take_i32(r); c->kw = take_i32(r);
    c->pad = take_i32(r); c->stride = take_i32(r);
    if (r->bad) return;
    if (c->tag == TAG_BIN) {
        c->nwords = take_i32(r);
        size_t n = count_or_fail(r, c->cout, c->nwords, 1, 1, 8);
        c->bits = take(r, n * 8);
    } else if (c->tag == TAG_REAL) {
        size_t n = count_or_fail(r, c->cout, c->cin, c->kh, c->kw, 1);
        c->wsign = take(r, n);
        size_t na = count_or_fail(r, c->cout, 1, 1, 1, 4);
        c->alpha = take(r, na * 4);
    } else {
        fail(r, "bad conv tag %d", c->tag);
    }
}

static void parse_act(reader *r, orc_act *a) {
    memset(a, 0, sizeof *a);
    int tag = take_i32(r);
    if (!r->bad && tag != TAG_ACT) { fail(r, "bad act tag %d", tag); return; }
    a->kind = take_i32(r);
    a->c = take_i32(r);
    count_or_fail(r, a->c, 4, 1, 1, 4);       /* four arrays of C x 4 bytes */
    const size_t n = r->bad ? 0 : (size_t)a->c;
    if (r->bad) return;
    if (a->kind == 0) {          /* any other kind is the real fold (csrc/bnn_model.c:114-124) */
        a->type = take(r, n * 4); a->t = take(r, n * 4);
        a->lo = take(r, n * 4); a->hi = take(r, n * 4);
    } else {
        a->A = take(r, n * 4); a->B = take(r, n * 4);
        a->slope = take(r, n * 4); a->rsign = take(r, n * 4);
    }
}

static void free_conv(orc_conv *c) { free(c->bits); free(c->wsign); free(c->alpha); }
static void free_act(orc_act *a) {
    free(a->type); free(a->t); free(a->lo); free(a->hi);
    free(a->A); free(a->B); free(a->slope); free(a->rsign);
}

void orc_free(orc_model *m) {
    if (!m) return;
    for (int i = 0; i < 4; ++i) {
        free_conv(&m->enc_c1[i]); free_conv(&m->enc_c2[i]);
        free_act(&m->enc_a1[i]); free_act(&m->enc_skip[i]); free_act(&m->enc_down[i]);
        free_conv(&m->dec_c1[i]); free_conv(&m->dec_c2[i]);
        free_act(&m->dec_a1[i]); free_act(&m->dec_a2[i]);
    }
    free_conv(&m->bott_c1); free_conv(&m->bott_c2);
    free_act(&m->bott_a1); free_act(&m->bott_a2);
    free_conv(&m->stem_c); free_act(&m->stem_a);
    free(m->head_w); free(m->head_b);
    free(m);
}

int orc_parse(const uint8_t *buf, size_t len, int strict, orc_model **out,
              char *err, int errlen) {
    reader r = {buf, len, 0, err, errlen, 0};
    *out = NULL;
    if (len < 4) { fail(&r, "short read"); return 1; }
    if (memcmp(buf, "BNNC", 4) != 0) { fail(&r, "bad magic"); return 1; }
    r.o = 4;
    orc_model *m = calloc(1, sizeof *m);
    if (!m) { fail(&r, "out of memory"); return 1; }
    m->version = take_i32(&r); m->base = take_i32(&r);
    m->n_bands = take_i32(&r); m->n_classes = take_i32(&r);
    m->upsampler = take_i32(&r);
    if (!r.bad && strict && m->version != 1 && m->version != 2)
        fail(&r, "unsupported blob version %d", m->version);
    if (!r.bad && strict && m->upsampler != 0) fail(&r, "unsupported upsampler %d", m->upsampler);
    if (!r.bad && m->version == 2) {
        /* <7i> header and the stem records (csrc/bnn_model_stem.c:86-96) */
        m->has_stem = take_i32(&r); m->n_stem_layers = take_i32(&r);
        if (!r.bad && (m->has_stem != 1 || m->n_stem_layers != 1))
            fail(&r, "only has_stem=1, n_stem_layers=1 supported");
        parse_conv(&r, &m->stem_c); parse_act(&r, &m->stem_a);
    }
    for (int i = 0; i < 4; ++i) {
        parse_conv(&r, &m->enc_c1[i]); parse_act(&r, &m->enc_a1[i]);
        parse_conv(&r, &m->enc_c2[i]); parse_act(&r, &m->enc_skip[i]);
        parse_act(&r, &m->enc_down[i]);
    }
    parse_conv(&r, &m->bott_c1); parse_act(&r, &m->bott_a1);
    parse_conv(&r, &m->bott_c2); parse_act(&r, &m->bott_a2);
    for (int i = 0; i < 4; ++i) {
        parse_conv(&r, &m->dec_c1[i]); parse_act(&r, &m->dec_a1[i]);
        parse_conv(&r, &m->dec_c2[i]); parse_act(&r, &m->dec_a2[i]);
    }
    int tag = take_i32(&r);
    if (!r.bad && tag != TAG_HEAD) fail(&r, "bad head tag %d", tag);
    m->head_cout = take_i32(&r); m->head_cin = take_i32(&r);
    size_t nw = count_or_fail(&r, m->head_cout, m->head_cin, 1, 1, 4);
    m->head_w = take(&r, nw * 4);
    size_t nb = count_or_fail(&r, m->head_cout, 1, 1, 1, 4);
    m->head_b = take(&r, nb * 4);
    if (!r.bad && r.o != r.n) fail(&r, "trailing bytes in blob");
    if (r.bad) { orc_free(m); return 1; }
    *out = m;
    return 0;
}

/* ---------------------------------------------------------- binary conv */
static int out_size(int in, int k, int pad, int stride) {
    return (in + 2 * pad - k) / stride + 1;
}

void orc_pack_kidx(const int8_t *wsign, uint64_t *bits, int cout, int cin,
                   int kh, int kw) {
    /* csrc/bnn_conv.c:80-95: kidx = (ci*kh+ky)*kw+kx is the C-order index of
     * wsign[co], bit set iff w > 0, LSB-first within 64-bit words. */
    const int K = cin * kh * kw, nw = (K + 63) / 64;
    for (int co = 0; co < cout; ++co) {
        uint64_t *dst = bits + (size_t)co * nw;
        memset(dst, 0, (size_t)nw * 8);
        const int8_t *src = wsign + (size_t)co * K;
        for (int k = 0; k < K; ++k)
            if (src[k] > 0) dst[k >> 6] |= 1ull << (k & 63);
    }
}

/* P = sum over in-bounds taps of a*w; padded taps contribute 0
 * (csrc/bnn_conv.c:50-76, the reference's +-1 triple-loop oracle). */
void orc_bconv_naive(const int8_t *a, const int8_t *wsign, int32_t *P, int cin,
                     int H, int W, int cout, int kh, int kw, int pad, int stride) {
    const int Ho = out_size(H, kh, pad, stride), Wo = out_size(W, kw, pad, stride);
    for (int co = 0; co < cout; ++co)
        for (int oy = 0; oy < Ho; ++oy)
            for (int ox = 0; ox < Wo; ++ox) {
                int32_t sum = 0;
                for (int ci = 0; ci < cin; ++ci)
                    for (int ky = 0; ky < kh; ++ky) {
                        const int iy = oy * stride + ky - pad;
                        if (iy < 0 || iy >= H) continue;
                        for (int kx = 0; kx < kw; ++kx) {
                            const int ix = ox * stride + kx - pad;
                            if (ix < 0 || ix >= W) continue;
                            sum += (int32_t)wsign[(((size_t)co * cin + ci) * kh + ky) * kw + kx] *
                                   (int32_t)a[((size_t)ci * H + iy) * W + ix];
                        }
                    }
                P[((size_t)co * Ho + oy) * Wo + ox] = sum;
            }
}

/* Dense kidx form (csrc/bnn_conv.c:99-142): per output pixel gather the
 * receptive field into a kidx bit vector plus a validity mask, then
 * P = 2*popcount(XNOR(w,a) & valid) - popcount(valid).  An activation <= 0
 * is a 0 bit (-1); only out-of-image taps are masked. */
void orc_bconv_dense(const int8_t *a, const uint64_t *bits, int32_t *P, int cin,
                     int H, int W, int cout, int kh, int kw, int pad, int stride) {
    const int Ho = out_size(H, kh, pad, stride), Wo = out_size(W, kw, pad, stride);
    const int K = cin * kh * kw, nw = (K + 63) / 64;
    #pragma omp parallel for schedule(static)
    for (int oy = 0; oy < Ho; ++oy) {
        uint64_t *act = malloc((size_t)nw * 16), *valid = act + nw;
        for (int ox = 0; ox < Wo; ++ox) {
            memset(act, 0, (size_t)nw * 16);
            int k = 0;
            for (int ci = 0; ci < cin; ++ci)
                for (int ky = 0; ky < kh; ++ky)
                    for (int kx = 0; kx < kw; ++kx, ++k) {
                        const int iy = oy * stride + ky - pad, ix = ox * stride + kx - pad;
                        if (iy < 0 || iy >= H || ix < 0 || ix >= W) continue;
                        valid[k >> 6] |= 1ull << (k & 63);
                        if (a[((size_t)ci * H + iy) * W + ix] > 0) act[k >> 6] |= 1ull << (k & 63);
                    }
            int nvalid = 0;
            for (int j = 0; j < nw; ++j) nvalid += __builtin_popcountll(valid[j]);
            for (int co = 0; co < cout; ++co) {
                const uint64_t *wr = bits + (size_t)co * nw;
                int eq = 0;
                for (int j = 0; j < nw; ++j) eq += __builtin_popcountll(~(wr[j] ^ act[j]) & valid[j]);
                P[((size_t)co * Ho + oy) * Wo + ox] = 2 * eq - nvalid;
            }
        }
        free(act);
    }
}

/* Channel-packed form (csrc/bnn_conv.c:144-213): activations packed once per
 * pixel along channels, weights regrouped per tap along channels, taps
 * clipped to the image, the last channel word masked to Cin. */
void orc_bconv_chan(const int8_t *a, const uint64_t *bits, int32_t *P, int cin,
                    int H, int W, int cout, int kh, int kw, int pad, int stride) {
    const int Ho = out_size(H, kh, pad, stride), Wo = out_size(W, kw, pad, stride);
    const int cw = (cin + 63) / 64, K = cin * kh * kw, nw = (K + 63) / 64;
    const uint64_t last = (cin & 63) ? ((1ull << (cin & 63)) - 1) : ~0ull;
    uint64_t *ap = calloc((size_t)H * W * cw + 1, 8);
    uint64_t *wp = calloc((size_t)cout * kh * kw * cw + 1, 8);
    if (!ap || !wp) { fprintf(stderr, "oracle: out of memory\n"); exit(1); }
    for (int ci = 0; ci < cin; ++ci)
        for (int p = 0; p < H * W; ++p)
            if (a[(size_t)ci * H * W + p] > 0) ap[(size_t)p * cw + (ci >> 6)] |= 1ull << (ci & 63);
    for (int co = 0; co < cout; ++co)
        for (int ci = 0; ci < cin; ++ci)
            for (int tap = 0; tap < kh * kw; ++tap) {
                const int k = ci * kh * kw + tap;
                if ((bits[(size_t)co * nw + (k >> 6)] >> (k & 63)) & 1)
                    wp[((size_t)co * kh * kw + tap) * cw + (ci >> 6)] |= 1ull << (ci & 63);
            }
    #pragma omp parallel for schedule(static)
    for (int oy = 0; oy < Ho; ++oy) {
        const int y0 = oy * stride - pad;
        const int ky0 = y0 < 0 ? -y0 : 0, ky1 = y0 + kh > H ? H - y0 : kh;
        for (int ox = 0; ox < Wo; ++ox) {
            const int x0 = ox * stride - pad;
            const int kx0 = x0 < 0 ? -x0 : 0, kx1 = x0 + kw > W ? W - x0 : kw;
            const int nvalid = (ky1 - ky0) * (kx1 - kx0) * cin;
            for (int co = 0; co < cout; ++co) {
                int eq = 0;
                for (int ky = ky0; ky < ky1; ++ky)
                    for (int kx = kx0; kx < kx1; ++kx) {
                        const uint64_t *av = ap + ((size_t)(y0 + ky) * W + (x0 + kx)) * cw;
                        const uint64_t *wv = wp + ((size_t)co * kh * kw + ky * kw + kx) * cw;
                        for (int j = 0; j < cw; ++j)
                            eq += __builtin_popcountll(~(av[j] ^ wv[j]) & (j == cw - 1 ? last : ~0ull));
                    }
                P[((size_t)co * Ho + oy) * Wo + ox] = 2 * eq - nvalid;
            }
        }
    }
    free(ap); free(wp);
}

/* csrc/bnn_conv.c:43-44, 216-223: channel-packed from Cin 36 up, dense below */
void orc_bconv(const int8_t *a, const uint64_t *bits, int32_t *P, int cin,
               int H, int W, int cout, int kh, int kw, int pad, int stride) {
    if (cin >= 36) orc_bconv_chan(a, bits, P, cin, H, W, cout, kh, kw, pad, stride);
    else orc_bconv_dense(a, bits, P, cin, H, W, cout, kh, kw, pad, stride);
}

/* ------------------------------------------------------ real-input conv */
/* csrc/bnn_conv_realin.c:66-116.  Per output (co,oy,ox): for every tap in
 * the clipped range, row-major, s = x*w summed over ci from 0 in order,
 * acc += s; out = alpha*acc.  Products with +-1 weights are exact.  The
 * channels of a block are separate chains advanced together, which leaves
 * each chain's order untouched. */
static void conv_real_general(const float *x, const int8_t *wsign, const float *alpha,
                              float *out, int cin, int H, int W, int cout, int kh,
                              int kw, int pad, int stride) {
    const int Ho = out_size(H, kh, pad, stride), Wo = out_size(W, kw, pad, stride);
    float *xt = malloc((size_t)H * W * cin * sizeof(float) + 4);
    float *wt = malloc((size_t)kh * kw * cin * cout * sizeof(float) + 4);
    if (!xt || !wt) { fprintf(stderr, "oracle: out of memory\n"); exit(1); }
    for (int ci = 0; ci < cin; ++ci)
        for (int p = 0; p < H * W; ++p) xt[(size_t)p * cin + ci] = x[(size_t)ci * H * W + p];
    for (int co = 0; co < cout; ++co)
        for (int ci = 0; ci < cin; ++ci)
            for (int tap = 0; tap < kh * kw; ++tap)
                wt[((size_t)tap * cin + ci) * cout + co] =
                    (float)wsign[((size_t)co * cin + ci) * kh * kw + tap];
    /* output rows in parallel: each output is still one thread's chain */
    #pragma omp parallel
    {
    float *acc = malloc((size_t)cout * 2 * sizeof(float) + 8), *s = acc + cout;
    if (!acc) { fprintf(stderr, "oracle: out of memory\n"); exit(1); }
    #pragma omp for schedule(static)
    for (int oy = 0; oy < Ho; ++oy) {
        const int y0 = oy * stride - pad;
        const int ky0 = y0 < 0 ? -y0 : 0, ky1 = y0 + kh > H ? H - y0 : kh;
        for (int ox = 0; ox < Wo; ++ox) {
            const int x0 = ox * stride - pad;
            const int kx0 = x0 < 0 ? -x0 : 0, kx1 = x0 + kw > W ? W - x0 : kw;
            for (int co = 0; co < cout; ++co) acc[co] = 0.0f;
            for (int ky = ky0; ky < ky1; ++ky)
                for (int kx = kx0; kx < kx1; ++kx) {
                    const float *xv = xt + ((size_t)(y0 + ky) * W + (x0 + kx)) * cin;
                    const float *wv = wt + (size_t)(ky * kw + kx) * cin * cout;
                    for (int co = 0; co < cout; ++co) s[co] = 0.0f;
                    for (int ci = 0; ci < cin; ++ci) {
                        const float xc = xv[ci];
                        const float *wr = wv + (size_t)ci * cout;
                        for (int co = 0; co < cout; ++co) s[co] = s[co] + xc * wr[co];
                    }
                    for (int co = 0; co < cout; ++co) acc[co] = acc[co] + s[co];
                }
            for (int co = 0; co < cout; ++co)
                out[((size_t)co * Ho + oy) * Wo + ox] = alpha[co] * acc[co];
        }
    }
    free(acc);
    }
    free(xt); free(wt);
}

/* csrc/bnn_conv_realin.c:140-155: 1x1/pad 0/stride 1 as Cin rank-1 updates
 * over the pixel plane, then the alpha scale. */
static void conv_real_1x1(const float *x, const int8_t *wsign, const float *alpha,
                          float *out, int cin, int H, int W, int cout) {
    const size_t hw = (size_t)H * W;
    for (int co = 0; co < cout; ++co) {
        float *o = out + co * hw;
        for (size_t p = 0; p < hw; ++p) o[p] = 0.0f;
        for (int ci = 0; ci < cin; ++ci) {
            const float wv = (float)wsign[(size_t)co * cin + ci];
            const float *xr = x + ci * hw;
            for (size_t p = 0; p < hw; ++p) o[p] = o[p] + wv * xr[p];
        }
        for (size_t p = 0; p < hw; ++p) o[p] = o[p] * alpha[co];
    }
}

void orc_conv_real(const float *x, const int8_t *wsign, const float *alpha,
                   float *out, int cin, int H, int W, int cout, int kh, int kw,
                   int pad, int stride) {
    /* csrc/bnn_conv_realin.c:165-172 */
    if (kh == 1 && kw == 1 && pad == 0 && stride == 1)
        conv_real_1x1(x, wsign, alpha, out, cin, H, W, cout);
    else
        conv_real_general(x, wsign, alpha, out, cin, H, W, cout, kh, kw, pad, stride);
}

/* ----------------------------------------------------------------- folds */
/* csrc/bnn_fold.c:37-60 */
void orc_fold_int(const int32_t *P, int8_t *out, int C, int H, int W,
                  const int32_t *type, const int32_t *t, const int32_t *lo,
                  const int32_t *hi) {
    const size_t hw = (size_t)H * W;
    for (int c = 0; c < C; ++c) {
        const int32_t *p = P + c * hw;
        int8_t *o = out + c * hw;
        for (size_t i = 0; i < hw; ++i) {
            const int32_t v = p[i];
            int on;
            switch (type[c]) {
            case 0: on = t[c] > 0; break;
            case 1: on = v >= t[c]; break;
            case 2: on = v < t[c]; break;
            case 3: on = v >= lo[c] && v < hi[c]; break;
            case 4: on = v < lo[c] || v >= hi[c]; break;
            default: on = 0; break;
            }
            o[i] = on ? 1 : -1;
        }
    }
}

/* csrc/bnn_fold.c:62-77, with the reference build's contraction of A*x+B */
void orc_fold_real(const float *x, int8_t *out, int C, int H, int W,
                   const float *A, const float *B, const float *slope,
                   const float *rsign) {
    const size_t hw = (size_t)H * W;
    for (int c = 0; c < C; ++c)
        for (size_t i = 0; i < hw; ++i) {
            float z = fmaf(A[c], x[c * hw + i], B[c]);
            if (z < 0.0f) z = slope[c] * z;
            const float r = z + rsign[c];
            out[c * hw + i] = r > 0.0f ? 1 : -1;
        }
}

/* --------------------------------------------------------- pool / head */
/* csrc/bnn_maxpool.c:28-48: floor-mode k x k max over int32 P */
void orc_maxpool(const int32_t *P, int32_t *out, int C, int H, int W, int k,
                 int stride) {
    const int Ho = (H - k) / stride + 1, Wo = (W - k) / stride + 1;
    for (int c = 0; c < C; ++c)
        for (int oy = 0; oy < Ho; ++oy)
            for (int ox = 0; ox < Wo; ++ox) {
                int32_t m = INT32_MIN;
                for (int dy = 0; dy < k; ++dy)
                    for (int dx = 0; dx < k; ++dx) {
                        const int32_t v = P[((size_t)c * H + oy * stride + dy) * W + ox * stride + dx];
                        if (v > m) m = v;
                    }
                out[((size_t)c * Ho + oy) * Wo + ox] = m;
            }
}

/* csrc/bnn_head.c:21-34: logits = bias then += W*a for c ascending; the
 * reference build fuses each step (vfmadd231ss). */
void orc_head(const float *a, const float *Wt, const float *bias, float *logits,
              int cin, int H, int W, int cout) {
    const size_t hw = (size_t)H * W;
    for (int o = 0; o < cout; ++o)
        for (size_t p = 0; p < hw; ++p) {
            float acc = bias[o];
            for (int c = 0; c < cin; ++c) acc = fmaf(Wt[(size_t)o * cin + c], a[c * hw + p], acc);
            logits[o * hw + p] = acc;
        }
}

/* csrc/bnn_model.c:130-148: [skip ; nearest-2x(x) placed at the F.pad
 * before-offset], positions the upsample does not reach stay 0. */
void orc_up_cat(const int8_t *skip, int sC, int sH, int sW, const int8_t *x,
                int xC, int hH, int hW, int8_t *out) {
    memset(out, 0, (size_t)(sC + xC) * sH * sW);
    memcpy(out, skip, (size_t)sC * sH * sW);
    const int uH = 2 * hH, uW = 2 * hW;
    const int oh = sH > uH ? (sH - uH) / 2 : 0, ow = sW > uW ? (sW - uW) / 2 : 0;
    const int nH = uH < sH ? uH : sH, nW = uW < sW ? uW : sW;
    for (int c = 0; c < xC; ++c)
        for (int y = 0; y < nH; ++y)
            for (int xx = 0; xx < nW; ++xx)
                out[((size_t)(sC + c) * sH + oh + y) * sW + ow + xx] =
                    x[((size_t)c * hH + y / 2) * hW + xx / 2];
}

/* --------------------------------------------------------------- forward */
static int conv_ok(const orc_conv *c, int tag, int cin) {
    return c->tag == tag && c->cin == cin && c->cout > 0 && c->kh == 3 && c->kw == 3 &&
           c->pad == 1 && c->stride == 1 &&
           (tag != TAG_BIN || c->nwords == (cin * 9 + 63) / 64);
}
static int act_ok(const orc_act *a, int kind, int c) {
    return a->c == c && (kind ? a->kind != 0 : a->kind == 0);
}

/* The topology checks a valid v1 blob always passes; the reference trusts
 * the blob instead (csrc/bnn_model.c:150-253). */
static int model_ok(const orc_model *m, int H, int W) {
    if (H < 16 || W < 16) return 0;            /* four 2x2 pools need >= 1 pixel */
    if (m->n_bands <= 0 || m->n_classes <= 0) return 0;
    int c = m->n_bands;
    const int stem = m->has_stem;
    if (stem) {
        const orc_conv *s = &m->stem_c;
        if (s->tag != TAG_REAL || s->cin != c || s->cout <= 0 || s->kh != 1 || s->kw != 1 ||
            s->pad != 0 || s->stride != 1 || !act_ok(&m->stem_a, 1, s->cout)) return 0;
        c = s->cout;
    }
    int skipc[4];
    for (int i = 0; i < 4; ++i) {
        const orc_conv *c1 = &m->enc_c1[i], *c2 = &m->enc_c2[i];
        const int real = i == 0 && !stem;
        if (!conv_ok(c1, real ? TAG_REAL : TAG_BIN, c)) return 0;
        if (!act_ok(&m->enc_a1[i], real, c1->cout)) return 0;
        if (!conv_ok(c2, TAG_BIN, c1->cout)) return 0;
        if (!act_ok(&m->enc_skip[i], 0, c2->cout) || !act_ok(&m->enc_down[i], 0, c2->cout)) return 0;
        skipc[i] = c = c2->cout;
    }
    if (!conv_ok(&m->bott_c1, TAG_BIN, c) || !act_ok(&m->bott_a1, 0, m->bott_c1.cout)) return 0;
    c = m->bott_c1.cout;
    if (!conv_ok(&m->bott_c2, TAG_BIN, c) || !act_ok(&m->bott_a2, 0, m->bott_c2.cout)) return 0;
    c = m->bott_c2.cout;
    for (int i = 0; i < 4; ++i) {
        const orc_conv *c1 = &m->dec_c1[i], *c2 = &m->dec_c2[i];
        if (!conv_ok(c1, TAG_BIN, skipc[3 - i] + c) || !act_ok(&m->dec_a1[i], 0, c1->cout)) return 0;
        if (!conv_ok(c2, TAG_BIN, c1->cout) || !act_ok(&m->dec_a2[i], 0, c2->cout)) return 0;
        c = c2->cout;
    }
    return m->head_cin == c && m->head_cout == m->n_classes;
}

static void emit(orc_stage_cb cb, void *ctx, const char *name, int dtype, int c,
                 int h, int w, const void *data) {
    if (cb) cb(ctx, name, dtype, c, h, w, data);
}

static void *xalloc(size_t n) {
    void *p = malloc(n ? n : 1);
    if (!p) { fprintf(stderr, "oracle: out of memory\n"); exit(1); }
    return p;
}

/* integer rule on P with a stage record for P and for the output */
static int8_t *conv_fold(const orc_conv *cv, const orc_act *ac, const int8_t *in,
                         int H, int W, const char *stage, const char *actname,
                         orc_stage_cb cb, void *ctx) {
    char nm[48];
    int32_t *P = xalloc((size_t)cv->cout * H * W * 4);
    orc_bconv(in, cv->bits, P, cv->cin, H, W, cv->cout, 3, 3, 1, 1);
    snprintf(nm, sizeof nm, "%s.P", stage);
    emit(cb, ctx, nm, 1, cv->cout, H, W, P);
    int8_t *out = xalloc((size_t)cv->cout * H * W);
    orc_fold_int(P, out, cv->cout, H, W, ac->type, ac->t, ac->lo, ac->hi);
    emit(cb, ctx, actname, 0, cv->cout, H, W, out);
    free(P);
    return out;
}

int orc_forward(const orc_model *m, const float *in, int H, int W, float *logits,
                orc_stage_cb cb, void *ctx) {
    if (!model_ok(m, H, W)) return 1;
    char nm[48], nm2[48];
    int8_t *skip[4];
    int sC[4], sH[4], sW[4];
    int8_t *x;
    int xC, xH = H, xW = W;

    if (m->has_stem) {
        /* v2: 1x1 real stem -> real fold (csrc/bnn_model_stem.c:175-190) */
        const orc_conv *sc = &m->stem_c;
        float *r = xalloc((size_t)sc->cout * H * W * 4);
        orc_conv_real(in, sc->wsign, sc->alpha, r, sc->cin, H, W, sc->cout, 1, 1, 0, 1);
        emit(cb, ctx, "stem.conv", 2, sc->cout, H, W, r);
        x = xalloc((size_t)sc->cout * H * W);
        orc_fold_real(r, x, sc->cout, H, W, m->stem_a.A, m->stem_a.B, m->stem_a.slope, m->stem_a.rsign);
        emit(cb, ctx, "stem.act", 0, sc->cout, H, W, x);
        free(r);
        xC = sc->cout;
    } else {
        /* v1 enc1: real conv -> real fold, then conv2 with two consumers */
        const orc_conv *c1 = &m->enc_c1[0], *c2 = &m->enc_c2[0];
        float *r = xalloc((size_t)c1->cout * H * W * 4);
        orc_conv_real(in, c1->wsign, c1->alpha, r, c1->cin, H, W, c1->cout, 3, 3, 1, 1);
        emit(cb, ctx, "enc1.conv1", 2, c1->cout, H, W, r);
        const orc_act *a1 = &m->enc_a1[0];
        x = xalloc((size_t)c1->cout * H * W);
        orc_fold_real(r, x, c1->cout, H, W, a1->A, a1->B, a1->slope, a1->rsign);
        emit(cb, ctx, "enc1.act1", 0, c1->cout, H, W, x);
        free(r);
        xC = c1->cout;
        (void)c2;
    }
    for (int i = 0; i < 4; ++i) {
        int8_t *h;
        if (i == 0 && !m->has_stem) {
            h = x;
        } else {
            snprintf(nm, sizeof nm, "enc%d.conv1", i + 1);
            snprintf(nm2, sizeof nm2, "enc%d.act1", i + 1);
            h = conv_fold(&m->enc_c1[i], &m->enc_a1[i], x, xH, xW, nm, nm2, cb, ctx);
            free(x);
        }
        const orc_conv *c2 = &m->enc_c2[i];
        int32_t *P = xalloc((size_t)c2->cout * xH * xW * 4);
        orc_bconv(h, c2->bits, P, c2->cin, xH, xW, c2->cout, 3, 3, 1, 1);
        snprintf(nm, sizeof nm, "enc%d.conv2.P", i + 1);
        emit(cb, ctx, nm, 1, c2->cout, xH, xW, P);
        free(h);
        const orc_act *as = &m->enc_skip[i], *ad = &m->enc_down[i];
        skip[i] = xalloc((size_t)c2->cout * xH * xW);
        orc_fold_int(P, skip[i], c2->cout, xH, xW, as->type, as->t, as->lo, as->hi);
        snprintf(nm, sizeof nm, "enc%d.act2_skip", i + 1);
        emit(cb, ctx, nm, 0, c2->cout, xH, xW, skip[i]);
        sC[i] = c2->cout; sH[i] = xH; sW[i] = xW;
        const int hH = xH / 2, hW = xW / 2;
        int32_t *Pd = xalloc((size_t)c2->cout * hH * hW * 4);
        orc_maxpool(P, Pd, c2->cout, xH, xW, 2, 2);
        snprintf(nm, sizeof nm, "enc%d.pool.P", i + 1);
        emit(cb, ctx, nm, 1, c2->cout, hH, hW, Pd);
        free(P);
        x = xalloc((size_t)c2->cout * hH * hW);
        orc_fold_int(Pd, x, c2->cout, hH, hW, ad->type, ad->t, ad->lo, ad->hi);
        snprintf(nm, sizeof nm, "enc%d.act2_down", i + 1);
        emit(cb, ctx, nm, 0, c2->cout, hH, hW, x);
        free(Pd);
        xC = c2->cout; xH = hH; xW = hW;
    }
    {
        int8_t *h = conv_fold(&m->bott_c1, &m->bott_a1, x, xH, xW, "bott.conv1", "bott.act1", cb, ctx);
        free(x);
        x = conv_fold(&m->bott_c2, &m->bott_a2, h, xH, xW, "bott.conv2", "bott.act2", cb, ctx);
        free(h);
        xC = m->bott_c2.cout;
    }
    for (int i = 0; i < 4; ++i) {
        const int si = 3 - i, st = 4 - i;
        const int cC = sC[si] + xC;
        int8_t *cat = xalloc((size_t)cC * sH[si] * sW[si]);
        orc_up_cat(skip[si], sC[si], sH[si], sW[si], x, xC, xH, xW, cat);
        snprintf(nm, sizeof nm, "dec%d.upcat", st);
        emit(cb, ctx, nm, 0, cC, sH[si], sW[si], cat);
        free(x); free(skip[si]);
        snprintf(nm, sizeof nm, "dec%d.conv1", st);
        snprintf(nm2, sizeof nm2, "dec%d.act1", st);
        int8_t *h = conv_fold(&m->dec_c1[i], &m->dec_a1[i], cat, sH[si], sW[si], nm, nm2, cb, ctx);
        free(cat);
        snprintf(nm, sizeof nm, "dec%d.conv2", st);
        snprintf(nm2, sizeof nm2, "dec%d.act2", st);
        x = conv_fold(&m->dec_c2[i], &m->dec_a2[i], h, sH[si], sW[si], nm, nm2, cb, ctx);
        free(h);
        xC = m->dec_c2[i].cout; xH = sH[si]; xW = sW[si];
    }
    {
        /* widen +-1 to float (exact), then the head (csrc/bnn_model.c:241-251) */
        const size_t n = (size_t)xC * xH * xW;
        float *xf = xalloc(n * 4);
        for (size_t j = 0; j < n; ++j) xf[j] = (float)x[j];
        orc_head(xf, m->head_w, m->head_b, logits, m->head_cin, xH, xW, m->head_cout);
        emit(cb, ctx, "logits", 2, m->head_cout, xH, xW, logits);
        free(xf);
    }
    free(x);
    return 0;
}

int orc_forward_batch(const orc_model *m, const float *in, int N, int H, int W,
                      float *logits) {
    const size_t is = (size_t)m->n_bands * H * W, os = (size_t)m->n_classes * H * W;
    for (int n = 0; n < N; ++n)
        if (orc_forward(m, in + n * is, H, W, logits + n * os, NULL, NULL)) return 1;
    return 0;
}

int orc_forward_batch_par(const orc_model *m, const float *in, int N, int H, int W,
                          float *logits) {
    if (!model_ok(m, H, W)) return 1;
    const size_t is = (size_t)m->n_bands * H * W, os = (size_t)m->n_classes * H * W;
    int bad = 0;
    #pragma omp parallel for schedule(dynamic, 1) reduction(| : bad)
    for (int n = 0; n < N; ++n)
        bad |= orc_forward(m, in + n * is, H, W, logits + n * os, NULL, NULL);
    return bad;
}
