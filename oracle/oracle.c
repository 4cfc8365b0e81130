/* CPU oracle for the newch hot path -- TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Restates, element by element and in the reference's evaluation order, what the reference engine
 * computes on x86-64 with its AVX2+FMA kernel tier.  Built with -ffp-contract=off: a product is
 * fused with an add only where fmaf() is written, which is exactly where the reference's AVX2 code
 * uses _mm256_fmadd_ps / _mm256_fnmadd_ps.  Everything else (the "scalar glue" of the ops files)
 * is plain IEEE single precision with the C association written in the reference source.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <stdint.h>
#include <string.h>

/* ---------------------------------------------------------------------------------------------- */
/* constants of the reference's published approximations                                          */
/* kernels_avx2.c:77-94 (Cephes expf polynomial, odd tanh series), :141-146 (A&S 7.1.26 erf),      */
/* ops_elementwise.c:216-219 (GELU)                                                                */
/* ---------------------------------------------------------------------------------------------- */
#define K_EXP_HI 88.8f
#define K_EXP_LO -87.3365448f
#define K_LOG2E 1.44269504088896341f
#define K_LN2_HI 0.693359375f
#define K_LN2_LO -2.12194440e-4f
#define K_EXP_P0 1.9875691500e-4f
#define K_EXP_P1 1.3981999507e-3f
#define K_EXP_P2 8.3334519073e-3f
#define K_EXP_P3 4.1665795894e-2f
#define K_EXP_P4 1.6666665459e-1f
#define K_EXP_P5 5.0000001201e-1f
#define K_TANH_SMALL 0.25f
#define K_TANH_T3 -0.333333333f
#define K_TANH_T5 0.133333333f
#define K_TANH_T7 -0.053968254f
#define K_TANH_T9 0.021869489f
#define K_ERF_P 0.3275911f
#define K_ERF_A1 0.254829592f
#define K_ERF_A2 -0.284496736f
#define K_ERF_A3 1.421413741f
#define K_ERF_A4 -1.453152027f
#define K_ERF_A5 1.061405429f
#define K_SQRT1_2 0.70710678118654752f
#define K_INV_SQRT_2PI 0.39894228040143268f
#define K_SQRT_2_PI 0.79788456080286536f
#define K_GELU_C 0.044715f

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* exp8, kernels_avx2.c:96-118.  max_ps/min_ps pick their second operand unless the first compares
 * greater/less, so a NaN input is clamped to LO and restored at the end. */
float or_exp(float x) {
    const float x0 = x;
    float xc = x > K_EXP_LO ? x : K_EXP_LO;
    xc = xc < K_EXP_HI ? xc : K_EXP_HI;
    float fx = floorf(fmaf(xc, K_LOG2E, 0.5f));
    float r = fmaf(-fx, K_LN2_HI, xc);
    r = fmaf(-fx, K_LN2_LO, r);
    float y = K_EXP_P0;
    y = fmaf(y, r, K_EXP_P1);
    y = fmaf(y, r, K_EXP_P2);
    y = fmaf(y, r, K_EXP_P3);
    y = fmaf(y, r, K_EXP_P4);
    y = fmaf(y, r, K_EXP_P5);
    y = fmaf(y, r * r, r + 1.0f);
    int32_t n = (int32_t)fx;
    int32_t big = n > 127;
    n -= big;
    float res = y * u2f((uint32_t)(n + 127) << 23);
    res = res * (big ? 2.0f : 1.0f);
    if (x0 < K_EXP_LO) res = 0.0f;
    if (x0 != x0) res = x0;
    return res;
}

/* sigmoid8, kernels_avx2.c:120-123 */
float or_sigmoid(float x) { return 1.0f / (1.0f + or_exp(0.0f - x)); }

/* tanh8, kernels_avx2.c:125-137 */
float or_tanh(float x) {
    const uint32_t sign = f2u(x) & 0x80000000u;
    float ax = u2f(f2u(x) & 0x7fffffffu);
    float e = or_exp(ax * -2.0f);
    float big = (1.0f - e) / (1.0f + e);
    big = u2f(f2u(big) | sign);
    float z = x * x;
    float p = fmaf(K_TANH_T9, z, K_TANH_T7);
    p = fmaf(p, z, K_TANH_T5);
    p = fmaf(p, z, K_TANH_T3);
    p = fmaf(p * z, x, x);
    return ax < K_TANH_SMALL ? p : big;
}

/* erf8, kernels_avx2.c:148-159 */
float or_erf(float x) {
    const uint32_t sign = f2u(x) & 0x80000000u;
    float ax = u2f(f2u(x) & 0x7fffffffu);
    float t = 1.0f / fmaf(ax, K_ERF_P, 1.0f);
    float p = fmaf(K_ERF_A5, t, K_ERF_A4);
    p = fmaf(p, t, K_ERF_A3);
    p = fmaf(p, t, K_ERF_A2);
    p = fmaf(p, t, K_ERF_A1);
    float e = or_exp(0.0f - ax * ax);
    float r = fmaf(-(p * t), e, 1.0f);
    return u2f(f2u(r) | sign);
}

void or_map(int fn, int64_t n, const float *x, float *y) {
    for (int64_t i = 0; i < n; i++) {
        float v = x[i];
        y[i] = fn == 0 ? or_exp(v) : fn == 1 ? or_sigmoid(v) : fn == 2 ? or_tanh(v) : or_erf(v);
    }
}

/* sum_f32, kernels_avx2.c:61-71 with hsum8 :12-17: two 8-lane accumulators over blocks of 16, lane
 * tree ((v0+v4)+(v2+v6))+((v1+v5)+(v3+v7)), then the tail added in order. */
float or_sum_f32(int64_t n, const float *x) {
    float a0[8] = {0}, a1[8] = {0};
    int64_t i = 0;
    for (; i + 16 <= n; i += 16) {
        for (int k = 0; k < 8; k++) {
            a0[k] = a0[k] + x[i + k];
            a1[k] = a1[k] + x[i + 8 + k];
        }
    }
    float v[8];
    for (int k = 0; k < 8; k++) v[k] = a0[k] + a1[k];
    float s = ((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7]));
    for (; i < n; i++) s = s + x[i];
    return s;
}

/* axpy_f32, kernels_avx2.c:39-45: y += alpha * x with a fused multiply-add */
void or_axpy(int64_t n, float alpha, const float *x, float *y) {
    for (int64_t i = 0; i < n; i++) y[i] = fmaf(alpha, x[i], y[i]);
}

/* ---------------------------------------------------------------------------------------------- */
/* activations: ops_elementwise.c:229-266 (forward), :289-338 (backward)                           */
/* ---------------------------------------------------------------------------------------------- */
void or_unary_fwd(int kind, float s, const float *x, float *y, int64_t n) {
    const float sixth = 1.0f / 6.0f;
    for (int64_t i = 0; i < n; i++) {
        float v = x[i], r;
        switch (kind) {
        case OR_UN_RELU: r = v > 0.0f ? v : 0.0f; break; /* relu_f32 = max_ps(x, 0) */
        case OR_UN_LEAKY_RELU: r = v > 0.0f ? v : s * v; break;
        case OR_UN_RELU6: r = fminf(fmaxf(v, 0.0f), 6.0f); break;
        case OR_UN_HARDSIGMOID: r = fminf(fmaxf(v * sixth + 0.5f, 0.0f), 1.0f); break;
        case OR_UN_HARDSWISH: r = (v * fminf(fmaxf(v + 3.0f, 0.0f), 6.0f)) * sixth; break;
        case OR_UN_SILU: r = or_sigmoid(v) * v; break;
        case OR_UN_GELU: r = (0.5f * v) * (1.0f + or_erf(K_SQRT1_2 * v)); break;
        case OR_UN_GELU_TANH: {
            float u = K_SQRT_2_PI * (v + ((K_GELU_C * v) * v) * v);
            r = (0.5f * v) * (1.0f + or_tanh(u));
            break;
        }
        case OR_UN_SIGMOID: r = or_sigmoid(v); break;
        case OR_UN_TANH: r = or_tanh(v); break;
        case OR_UN_EXP: r = or_exp(v); break;
        case OR_UN_NEG: r = -1.0f * v; break; /* scale_f32(-1) */
        case OR_UN_SCALE: r = s * v; break;
        case OR_UN_ADD_SCALAR: r = v + s; break;
        /* the reference's scalar libm calls (ops_elementwise.c:233-234, 240) */
        case OR_UN_LOG: r = logf(v); break;
        case OR_UN_SQRT: r = sqrtf(v); break;
        case OR_UN_POW: r = powf(v, s); break;
        default: r = NAN; break;
        }
        y[i] = r;
    }
}

void or_unary_bwd(int kind, float s, const float *x, const float *y, const float *g, float *gi, int64_t n) {
    const float sixth = 1.0f / 6.0f, third = 1.0f / 3.0f;
    for (int64_t i = 0; i < n; i++) {
        float v = x ? x[i] : 0.0f, gg = g[i], t;
        switch (kind) {
        case OR_UN_RELU: t = v > 0.0f ? gg : 0.0f; gi[i] = gi[i] + t; break;
        case OR_UN_LEAKY_RELU: t = v > 0.0f ? gg : s * gg; gi[i] = gi[i] + t; break;
        case OR_UN_RELU6: t = (v > 0.0f && v < 6.0f) ? gg : 0.0f; gi[i] = gi[i] + t; break;
        case OR_UN_HARDSIGMOID: t = (v > -3.0f && v < 3.0f) ? gg * sixth : 0.0f; gi[i] = gi[i] + t; break;
        case OR_UN_HARDSWISH:
            t = v < -3.0f ? 0.0f : v <= 3.0f ? gg * (v * third + 0.5f) : gg;
            gi[i] = gi[i] + t;
            break;
        case OR_UN_SILU: {
            float sg = or_sigmoid(v);
            t = (gg * sg) * (1.0f + v * (1.0f - sg));
            gi[i] = gi[i] + t;
            break;
        }
        case OR_UN_GELU: {
            float e = or_erf(K_SQRT1_2 * v);
            float q = or_exp((-0.5f * v) * v);
            t = gg * (0.5f * (1.0f + e) + (v * K_INV_SQRT_2PI) * q);
            gi[i] = gi[i] + t;
            break;
        }
        case OR_UN_GELU_TANH: {
            float th = or_tanh(K_SQRT_2_PI * (v + ((K_GELU_C * v) * v) * v));
            float dt = ((1.0f - th * th) * K_SQRT_2_PI) * (1.0f + ((3.0f * K_GELU_C) * v) * v);
            t = gg * (0.5f * (1.0f + th) + (0.5f * v) * dt);
            gi[i] = gi[i] + t;
            break;
        }
        case OR_UN_SIGMOID: t = (gg * y[i]) * (1.0f - y[i]); gi[i] = gi[i] + t; break;
        case OR_UN_TANH: t = gg * (1.0f - y[i] * y[i]); gi[i] = gi[i] + t; break;
        case OR_UN_EXP: t = gg * y[i]; gi[i] = gi[i] + t; break;
        case OR_UN_NEG: gi[i] = fmaf(-1.0f, gg, gi[i]); break;      /* axpy_f32(-1) */
        case OR_UN_SCALE: gi[i] = fmaf(s, gg, gi[i]); break;        /* axpy_f32(s) */
        case OR_UN_ADD_SCALAR: gi[i] = fmaf(1.0f, gg, gi[i]); break; /* axpy_f32(1) */
        /* ops_elementwise.c:305-306, 312: g / x, g * 0.5 / y, g * s * powf(x, s - 1), left to right */
        case OR_UN_LOG: t = gg / v; gi[i] = gi[i] + t; break;
        case OR_UN_SQRT: t = (gg * 0.5f) / y[i]; gi[i] = gi[i] + t; break;
        case OR_UN_POW: t = (gg * s) * powf(v, s - 1.0f); gi[i] = gi[i] + t; break;
        default: gi[i] = NAN; break;
        }
    }
}

/* ---------------------------------------------------------------------------------------------- */
/* broadcasting: tensor.c:75-90 (broadcast strides), :313-345 (row-major odometer iteration)        */
/* ---------------------------------------------------------------------------------------------- */
#define OR_MAX_DIMS 6

static void contig_strides(int nd, const int64_t *shape, int64_t *st) {
    int64_t s = 1;
    for (int i = nd - 1; i >= 0; i--) { st[i] = s; s *= shape[i]; }
}

/* strides of a tensor (shape tshape, strides tst) broadcast onto an nd-d output shape */
static void bcast(int tn, const int64_t *tshape, const int64_t *tst, int nd, const int64_t *shape, int64_t *out) {
    for (int i = 0; i < nd; i++) {
        int j = i - (nd - tn);
        out[i] = (j < 0 || (tshape[j] == 1 && shape[i] != 1)) ? 0 : tst[j];
    }
}

static int64_t numel(int nd, const int64_t *shape) {
    int64_t n = 1;
    for (int i = 0; i < nd; i++) n *= shape[i];
    return n;
}

/* visits every output element in row-major order, giving the element offset of each operand */
typedef void (*visit_fn)(const int64_t *off, void *user);
static void visit(int nops, const int64_t (*st)[OR_MAX_DIMS], int nd, const int64_t *shape, visit_fn fn,
                  void *user) {
    int64_t off[4] = {0, 0, 0, 0};
    if (nd == 0) { fn(off, user); return; }
    for (int d = 0; d < nd; d++)
        if (shape[d] == 0) return;
    int64_t idx[OR_MAX_DIMS] = {0};
    for (;;) {
        fn(off, user);
        int d = nd - 1;
        while (d >= 0) {
            idx[d]++;
            for (int k = 0; k < nops; k++) off[k] += st[k][d];
            if (idx[d] < shape[d]) break;
            for (int k = 0; k < nops; k++) off[k] -= st[k][d] * shape[d];
            idx[d] = 0;
            d--;
        }
        if (d < 0) return;
    }
}

typedef struct {
    int op;
    const float *a, *b;
    float *o;
} fwd_ctx;

static void fwd_visit(const int64_t *off, void *u) {
    fwd_ctx *c = (fwd_ctx *)u;
    float x = c->a[off[0]], y = c->b[off[1]], r;
    switch (c->op) {
    case OR_BIN_ADD: r = x + y; break;
    case OR_BIN_SUB: r = x - y; break;
    case OR_BIN_MUL: r = x * y; break;
    default: r = x / y; break;
    }
    c->o[off[2]] = r;
}

/* binary_fwd, ops_elementwise.c:108-127 with row_add..row_div :19-30 */
void or_binary_fwd(int op, int nd, const int64_t *shape, const float *a, const int64_t *sa, const float *b,
                   const int64_t *sb, float *o, const int64_t *so) {
    int64_t st[4][OR_MAX_DIMS];
    memcpy(st[0], sa, sizeof(int64_t) * (size_t)nd);
    memcpy(st[1], sb, sizeof(int64_t) * (size_t)nd);
    memcpy(st[2], so, sizeof(int64_t) * (size_t)nd);
    fwd_ctx c = {op, a, b, o};
    visit(3, (const int64_t(*)[OR_MAX_DIMS])st, nd, shape, fwd_visit, &c);
}

typedef struct {
    int mode; /* 0: gx += alpha*g  1: gx += g*other  2: gx += g/other  3: gx -= g*a/(b*b) */
    float alpha;
    const float *g, *p1, *p2;
    float *gx;
} bwd_ctx;

static void bwd_visit(const int64_t *off, void *u) {
    bwd_ctx *c = (bwd_ctx *)u;
    float g = c->g[off[0]];
    switch (c->mode) {
    case 0: { float t = c->alpha * g; c->gx[off[1]] = c->gx[off[1]] + t; break; }     /* row_acc :33-36 */
    case 1: { float t = g * c->p1[off[1]]; c->gx[off[2]] = c->gx[off[2]] + t; break; } /* row_acc_mul :38-41 */
    case 2: { float t = g / c->p1[off[1]]; c->gx[off[2]] = c->gx[off[2]] + t; break; } /* row_acc_div :43-46 */
    default: {                                                                         /* row_acc_div_b :48-54 */
        float bb = c->p2[off[2]];
        float t = (g * c->p1[off[1]]) / (bb * bb);
        c->gx[off[3]] = c->gx[off[3]] - t;
        break;
    }
    }
}

static int is_contig(int nd, const int64_t *shape, const int64_t *st) {
    int64_t s = 1;
    for (int i = nd - 1; i >= 0; i--) {
        if (shape[i] != 1 && st[i] != s) return 0;
        s *= shape[i];
    }
    return 1;
}

static int same_shape(int na, const int64_t *sa, int nb, const int64_t *sb) {
    if (na != nb) return 0;
    for (int i = 0; i < na; i++)
        if (sa[i] != sb[i]) return 0;
    return 1;
}

/* binary_bwd, ops_elementwise.c:129-186 */
void or_binary_bwd(int op, int a_nd, const int64_t *a_shape, const int64_t *a_stride, const float *a, int b_nd,
                   const int64_t *b_shape, const int64_t *b_stride, const float *b, const float *g, float *ga,
                   float *gb) {
    int nd = a_nd > b_nd ? a_nd : b_nd;
    int64_t shape[OR_MAX_DIMS] = {0}, so[OR_MAX_DIMS] = {0}, sa[OR_MAX_DIMS] = {0}, sb[OR_MAX_DIMS] = {0};
    for (int i = 0; i < nd; i++) {
        int ia = i - (nd - a_nd), ib = i - (nd - b_nd);
        int64_t da = ia < 0 ? 1 : a_shape[ia], db = ib < 0 ? 1 : b_shape[ib];
        shape[i] = da == 1 ? db : da;
    }
    contig_strides(nd, shape, so);
    bcast(a_nd, a_shape, a_stride, nd, shape, sa);
    bcast(b_nd, b_shape, b_stride, nd, shape, sb);
    const int64_t n = numel(nd, shape);
    const int flat = same_shape(a_nd, a_shape, nd, shape) && same_shape(b_nd, b_shape, nd, shape) &&
                     is_contig(a_nd, a_shape, a_stride) && is_contig(b_nd, b_shape, b_stride);
    for (int which = 0; which < 2; which++) {
        float *gx = which ? gb : ga;
        if (!gx) continue;
        int x_nd = which ? b_nd : a_nd;
        const int64_t *x_shape = which ? b_shape : a_shape;
        if (flat && op != OR_BIN_ADD && op != OR_BIN_SUB) {
            for (int64_t i = 0; i < n; i++) {
                float t;
                if (op == OR_BIN_MUL) { t = g[i] * (which ? a[i] : b[i]); gx[i] = gx[i] + t; }
                else if (which == 0) { t = g[i] / b[i]; gx[i] = gx[i] + t; }
                else { t = (g[i] * a[i]) / (b[i] * b[i]); gx[i] = gx[i] - t; }
            }
            continue;
        }
        int64_t xcs[OR_MAX_DIMS], sgx[OR_MAX_DIMS], st[4][OR_MAX_DIMS];
        contig_strides(x_nd, x_shape, xcs);
        bcast(x_nd, x_shape, xcs, nd, shape, sgx);
        memcpy(st[0], so, sizeof so);
        bwd_ctx c = {0, 1.0f, g, NULL, NULL, gx};
        if (op == OR_BIN_ADD || op == OR_BIN_SUB) {
            c.alpha = (op == OR_BIN_SUB && which == 1) ? -1.0f : 1.0f;
            if (same_shape(x_nd, x_shape, nd, shape)) {
                or_axpy(n, c.alpha, g, gx);
                continue;
            }
            c.mode = 0;
            memcpy(st[1], sgx, sizeof sgx);
            visit(2, (const int64_t(*)[OR_MAX_DIMS])st, nd, shape, bwd_visit, &c);
        } else if (op == OR_BIN_MUL || which == 0) {
            c.mode = op == OR_BIN_MUL ? 1 : 2;
            c.p1 = which == 0 ? b : a;
            memcpy(st[1], which == 0 ? sb : sa, sizeof sa);
            memcpy(st[2], sgx, sizeof sgx);
            visit(3, (const int64_t(*)[OR_MAX_DIMS])st, nd, shape, bwd_visit, &c);
        } else {
            c.mode = 3;
            c.p1 = a;
            c.p2 = b;
            memcpy(st[1], sa, sizeof sa);
            memcpy(st[2], sb, sizeof sb);
            memcpy(st[3], sgx, sizeof sgx);
            visit(4, (const int64_t(*)[OR_MAX_DIMS])st, nd, shape, bwd_visit, &c);
        }
    }
}

/* ---------------------------------------------------------------------------------------------- */
/* reductions: ops_reduce.c:60-163                                                                  */
/* ---------------------------------------------------------------------------------------------- */
void or_reduce_fwd(int kind, int64_t outer, int64_t R, int64_t inner, const float *x, float *y, int32_t *arg) {
    if (kind == OR_RED_SUM || kind == OR_RED_MEAN) {
        float scale = kind == OR_RED_MEAN ? 1.0f / (float)(R ? R : 1) : 1.0f;
        if (kind == OR_RED_MEAN && R == 0) {
            for (int64_t i = 0; i < outer * inner; i++) y[i] = NAN;
            return;
        }
        if (inner == 1) {
            for (int64_t o = 0; o < outer; o++) y[o] = scale * or_sum_f32(R, x + o * R);
            return;
        }
        memset(y, 0, (size_t)(outer * inner) * sizeof(float));
        for (int64_t o = 0; o < outer; o++)
            for (int64_t r = 0; r < R; r++) or_axpy(inner, scale, x + (o * R + r) * inner, y + o * inner);
        return;
    }
    for (int64_t o = 0; o < outer; o++) {
        for (int64_t i = 0; i < inner; i++) {
            const float *p = x + o * R * inner + i;
            int32_t best = 0;
            float bv = p[0];
            for (int64_t r = 1; r < R; r++)
                if (p[r * inner] > bv) { bv = p[r * inner]; best = (int32_t)r; }
            if (arg) arg[o * inner + i] = best;
            if (kind == OR_RED_MAX && y) y[o * inner + i] = bv;
        }
    }
}

void or_reduce_bwd(int kind, int64_t outer, int64_t R, int64_t inner, const float *g, const int32_t *arg,
                   float *gi) {
    if (kind == OR_RED_MAX) {
        for (int64_t o = 0; o < outer; o++)
            for (int64_t i = 0; i < inner; i++) {
                float *p = gi + (o * R + arg[o * inner + i]) * inner + i;
                *p = *p + g[o * inner + i];
            }
        return;
    }
    float scale = kind == OR_RED_MEAN ? 1.0f / (float)(R ? R : 1) : 1.0f;
    for (int64_t o = 0; o < outer; o++) {
        const float *gs = g + o * inner;
        if (inner == 1) {
            float v = scale * gs[0];
            for (int64_t r = 0; r < R; r++) gi[o * R + r] = gi[o * R + r] + v;
        } else {
            for (int64_t r = 0; r < R; r++) or_axpy(inner, scale, gs, gi + (o * R + r) * inner);
        }
    }
}

/* ---------------------------------------------------------------------------------------------- */
/* softmax / log_softmax: ops_nn.c:22-71                                                             */
/* ---------------------------------------------------------------------------------------------- */
void or_softmax_fwd(int log_form, int64_t rows, int64_t C, const float *x, float *y) {
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + r * C;
        float *yr = y + r * C;
        float m = xr[0];
        for (int64_t c = 1; c < C; c++)
            if (xr[c] > m) m = xr[c];
        for (int64_t c = 0; c < C; c++) yr[c] = or_exp(xr[c] - m);
        float s = or_sum_f32(C, yr);
        if (log_form) {
            float ls = logf(s);
            for (int64_t c = 0; c < C; c++) yr[c] = (xr[c] - m) - ls;
        } else {
            float inv = 1.0f / s;
            for (int64_t c = 0; c < C; c++) yr[c] = inv * yr[c];
        }
    }
}

void or_softmax_bwd(int log_form, int64_t rows, int64_t C, const float *y, const float *g, float *gi) {
    for (int64_t r = 0; r < rows; r++) {
        const float *yr = y + r * C, *gr = g + r * C;
        float *o = gi + r * C;
        if (log_form) {
            float sg = 0.0f;
            for (int64_t c = 0; c < C; c++) sg = sg + gr[c];
            for (int64_t c = 0; c < C; c++) {
                float t = expf(yr[c]) * sg;
                o[c] = o[c] + (gr[c] - t);
            }
        } else {
            float dot = 0.0f;
            for (int64_t c = 0; c < C; c++) { float t = gr[c] * yr[c]; dot = dot + t; }
            for (int64_t c = 0; c < C; c++) o[c] = o[c] + yr[c] * (gr[c] - dot);
        }
    }
}

/* ---------------------------------------------------------------------------------------------- */
/* layer norm: ops_nn.c:463-522 (fp64 row statistics, fp32 everything else)                         */
/* ---------------------------------------------------------------------------------------------- */
void or_layer_norm_fwd(int64_t rows, int64_t D, const float *x, const float *w, const float *b, float eps,
                       float *y, float *stats) {
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + r * D;
        double s = 0.0, ss = 0.0;
        for (int64_t i = 0; i < D; i++) s += xr[i];
        double mean = s / (double)D;
        for (int64_t i = 0; i < D; i++) { double d = xr[i] - mean; ss += d * d; }
        float rstd = (float)(1.0 / sqrt(ss / (double)D + eps));
        float meanf = (float)mean;
        stats[2 * r] = meanf;
        stats[2 * r + 1] = rstd;
        float *yr = y + r * D;
        for (int64_t i = 0; i < D; i++) {
            float v = (xr[i] - meanf) * rstd;
            float u = w ? v * w[i] : v;
            yr[i] = u + (b ? b[i] : 0.0f);
        }
    }
}

void or_layer_norm_bwd(int64_t rows, int64_t D, const float *x, const float *w, const float *stats,
                       const float *g, float *gx, float *gw, float *gb) {
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + r * D, *gr = g + r * D;
        float mean = stats[2 * r], rstd = stats[2 * r + 1];
        double sg = 0.0, sgx = 0.0;
        for (int64_t i = 0; i < D; i++) {
            float xhat = (xr[i] - mean) * rstd, gi = w ? gr[i] * w[i] : gr[i];
            sg += gi;
            float p = gi * xhat;
            sgx += p;
            if (gw) { float q = gr[i] * xhat; gw[i] = gw[i] + q; }
            if (gb) gb[i] = gb[i] + gr[i];
        }
        if (gx) {
            float *dx = gx + r * D, mg = (float)(sg / (double)D), mgx = (float)(sgx / (double)D);
            for (int64_t i = 0; i < D; i++) {
                float xhat = (xr[i] - mean) * rstd, gi = w ? gr[i] * w[i] : gr[i];
                float t = rstd * ((gi - mg) - xhat * mgx);
                dx[i] = dx[i] + t;
            }
        }
    }
}

/* ---------------------------------------------------------------------------------------------- */
/* int8: quantize_row ops_quant.c:11-21; dequantize = to_dtype i8->f32 (ops_shape.c:491-504, exact   */
/* through double) times the row scale (a broadcast mul, ops_elementwise.c:22 row_mul)               */
/* ---------------------------------------------------------------------------------------------- */
void or_quantize_rows(int64_t rows, int64_t cols, const float *w, int8_t *q, float *scale) {
    for (int64_t r = 0; r < rows; r++) {
        const float *x = w + r * cols;
        float amax = 0.0f;
        for (int64_t i = 0; i < cols; i++) amax = fmaxf(amax, fabsf(x[i]));
        float s = amax > 0.0f ? amax / 127.0f : 1.0f;
        float inv = 1.0f / s;
        for (int64_t i = 0; i < cols; i++) {
            float v = nearbyintf(x[i] * inv);
            float c = v > 127.0f ? 127.0f : v < -127.0f ? -127.0f : v;
            /* the reference's (int8_t) cast of a float goes through a 32-bit truncating conversion;
             * NaN (0/0 or inf*0 rows) converts to 0x80000000, whose low byte is 0 */
            q[r * cols + i] = c != c ? (int8_t)0 : (int8_t)(int32_t)c;
        }
        scale[r] = s;
    }
}

void or_dequantize_rows(int64_t rows, int64_t cols, const int8_t *q, const float *scale, float *w) {
    for (int64_t r = 0; r < rows; r++)
        for (int64_t i = 0; i < cols; i++) w[r * cols + i] = (float)(double)q[r * cols + i] * scale[r];
}

/* gemm_s8_nt (kernels_ref.c:117-128; the AVX2 tier kernels_avx2.c:314-340 sums the same products
 * in another order, exact either way): integer products summed in int64, stored as int32 (exact for
 * K <= 133143, where |C| <= K * 127 * 127 < 2^31). */
void or_gemm_s8_nt(int64_t M, int64_t N, int64_t K, const int8_t *A, int64_t lda, const int8_t *B, int64_t ldb,
                   int32_t *C, int64_t ldc) {
    for (int64_t i = 0; i < M; i++)
        for (int64_t j = 0; j < N; j++) {
            int64_t s = 0;
            for (int64_t k = 0; k < K; k++) s += (int32_t)A[i * lda + k] * (int32_t)B[j * ldb + k];
            C[i * ldc + j] = (int32_t)s;
        }
}

/* linear_int8 forward (ops_quant.c:72-113): each row of x quantized by quantize_row (:11-21), the
 * int8 product with wq, then the epilogue y = (float)acc * xs * ws + (bias or 0) of :75-79,
 * left to right, uncontracted. */
void or_linear_int8(int64_t M, int64_t K, int64_t N, const float *x, const int8_t *wq, const float *ws,
                    const float *bias, float *y) {
    int8_t *xq = (int8_t *)malloc((size_t)(M * K) + 1);
    float *xs = (float *)malloc((size_t)(M ? M : 1) * sizeof(float));
    int32_t *acc = (int32_t *)malloc((size_t)(M * N + 1) * sizeof(int32_t));
    or_quantize_rows(M, K, x, xq, xs);
    or_gemm_s8_nt(M, N, K, xq, K, wq, K, acc, N);
    for (int64_t r = 0; r < M; r++)
        for (int64_t o = 0; o < N; o++) {
            const float prod = (float)acc[r * N + o] * xs[r];
            y[r * N + o] = prod * ws[o] + (bias ? bias[o] : 0.0f);
        }
    free(xq);
    free(xs);
    free(acc);
}

/* ---------------------------------------------------------------------------------------------- */
/* cross entropy: ops_nn.c:107-147.  Per row the log-softmax of softmax_row (ops_nn.c:22-36), the  */
/* loss accumulated in double by subtraction in row order, then the row turned into probabilities  */
/* by the exp kernel (exp8 in the AVX2 tier); backward: gi += s * prob, gi[label] -= s.             */
/* ---------------------------------------------------------------------------------------------- */
int64_t or_cross_entropy_fwd(int64_t N, int64_t C, const float *x, const int32_t *lab, float *prob, float *loss) {
    double l = 0.0;
    for (int64_t i = 0; i < N; i++) {
        if (lab[i] < 0 || lab[i] >= C) return i;
        float *p = prob + i * C;
        or_softmax_fwd(1, 1, C, x + i * C, p);
        l -= p[lab[i]];
        for (int64_t c = 0; c < C; c++) p[c] = or_exp(p[c]);
    }
    *loss = N ? (float)(l / (double)N) : NAN;
    return -1;
}

void or_cross_entropy_bwd(int64_t N, int64_t C, const float *prob, const int32_t *lab, float gout, float *gi) {
    const float s = gout / (float)(N ? N : 1);
    for (int64_t i = 0; i < N; i++) {
        for (int64_t c = 0; c < C; c++) gi[i * C + c] = gi[i * C + c] + s * prob[i * C + c];
        gi[i * C + lab[i]] = gi[i * C + lab[i]] - s;
    }
}

/* ---------------------------------------------------------------------------------------------- */
/* nll loss: ops_nn.c:391-420 (double accumulation by subtraction in row order)                   */
/* ---------------------------------------------------------------------------------------------- */
int64_t or_nll_loss_fwd(int64_t N, int64_t C, const float *x, const int32_t *lab, int sum, float *loss) {
    double l = 0.0;
    for (int64_t i = 0; i < N; i++) {
        if (lab[i] < 0 || lab[i] >= C) return i;
        l -= x[i * C + lab[i]];
    }
    *loss = sum ? (float)l : N ? (float)(l / (double)N) : NAN;
    return -1;
}

void or_nll_loss_bwd(int64_t N, int64_t C, const int32_t *lab, float gout, int sum, float *gi) {
    const float s = sum ? gout : gout / (float)(N ? N : 1);
    for (int64_t i = 0; i < N; i++) gi[i * C + lab[i]] = gi[i * C + lab[i]] - s;
}

/* ---------------------------------------------------------------------------------------------- */
/* optimizers: optim.c:161-216 (scalar glue: fp32, left to right, no contraction); clip: :219-233  */
/* ---------------------------------------------------------------------------------------------- */
void or_optim_step(int kind, int64_t n, float *w, const float *g, float *s1, float *s2, float lr, float momentum,
                   float weight_decay, float beta1, float beta2, float eps, float gs, float bc1, float bc2,
                   int eps_inside_sqrt) {
    if (kind == OR_OPT_SGD) {
        for (int64_t j = 0; j < n; j++) {
            float gj = gs * g[j] + weight_decay * w[j];
            if (s1) gj = s1[j] = momentum * s1[j] + gj;
            w[j] -= lr * gj;
        }
    } else if (kind == OR_OPT_RMSPROP) {
        const float a = beta2;
        for (int64_t j = 0; j < n; j++) {
            float gj = gs * g[j] + weight_decay * w[j];
            s2[j] = a * s2[j] + (1.0f - a) * gj * gj;
            float den = eps_inside_sqrt ? sqrtf(s2[j] + eps) : sqrtf(s2[j]) + eps;
            float step = gj / den;
            if (s1) step = s1[j] = momentum * s1[j] + step;
            w[j] -= lr * step;
        }
    } else {
        const float l2 = kind == OR_OPT_ADAM ? weight_decay : 0.0f;
        const float decay = kind == OR_OPT_ADAMW ? 1.0f - lr * weight_decay : 1.0f;
        for (int64_t j = 0; j < n; j++) {
            w[j] *= decay;
            float gj = gs * g[j] + l2 * w[j];
            s1[j] = beta1 * s1[j] + (1.0f - beta1) * gj;
            s2[j] = beta2 * s2[j] + (1.0f - beta2) * gj * gj;
            w[j] -= lr * (s1[j] / bc1) / (sqrtf(s2[j] / bc2) + eps);
        }
    }
}

double or_sumsq(int64_t n, const float *x) {
    double ss = 0.0;
    for (int64_t j = 0; j < n; j++) ss += (double)x[j] * x[j];
    return ss;
}
