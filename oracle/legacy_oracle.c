/*
 * legacy_oracle.c -- CPU restatement of the reference's neuron-sparse fp16
 * FFN operator and activation predictor (the legacy sparse_moe C ABI).
 *
 * TEST INFRASTRUCTURE ONLY, like moe_oracle.c: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * What each function restates (paths relative to the reference root):
 *
 *   oracle_lg_predict      kernels/sparse_moe/gate_predict.cu:49-88 (gate =
 *                          sigmoid(w . x + b), mask = gate >= threshold) and
 *                          :153-177 (compaction in increasing neuron order),
 *                          driven as :200-242 drives them.
 *   oracle_lg_sparse_mlp   kernels/sparse_moe/sparse_matmul.cu:240-365: the
 *                          dense branch below 30% sparsity (:259-305: every
 *                          neuron, biases ignored), otherwise the sparse
 *                          branch (:306-364) with the reference grid's
 *                          coverage of list positions (:320-333), SwiGLU
 *                          (:120-146) and the down projection over the whole
 *                          list (:187-215).
 *   oracle_lg_sparsity     kernels/sparse_moe/gate_predict.cu:253-271.
 *
 * Two summation orders are restated for every dot product:
 *   order 0 (this build's contract, which the HIP kernels follow bit for bit)
 *     fp16 x fp16 products are exact in fp32.  Over D: 64 partial sums,
 *     partial l adding in increasing d, from +0.0, every product with
 *     (d mod 512) / 8 == l; partials combined by p[l] + p[l xor s] for
 *     s = 32, 16, 8, 4, 2, 1; then the bias (if any) added.  The down
 *     projection runs over the columns n of W_down with m_n, the number of
 *     times n appears among the first count list entries (every n once in
 *     the dense branch): columns with m_n = 0 are skipped, the others add
 *     fmaf(W[d, n], m_n * act[n], p) to partial l = (n mod 512) / 8 in
 *     increasing n; same tree.  This equals the sum over list entries in
 *     exact arithmetic.
 *   order 1 (the reference kernels' own loops)
 *     acc starts at the bias (or 0) and adds the products one at a time in
 *     increasing d, or in list order for the down projection
 *     (sparse_matmul.cu:80-96, :207-212; gate_predict.cu:71-74).
 * Sigmoid: order 0 uses (float)(1 / (1 + exp(-(double)a))); order 1 uses
 * the reference's fp32 expression 1.0f / (1.0f + expf(-a)) with this C
 * library's expf, which is not CUDA's expf, so order 1 is a close
 * restatement of the reference rather than a bit-exact one.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_API __attribute__((visibility("default")))

static float lg_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff, bits;
    if (e == 0) {
        float v = (float)m * (1.0f / 16777216.0f); /* exact: m * 2^-24 */
        memcpy(&bits, &v, 4);
        bits |= sign;
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* binary32 -> binary16, round to nearest even; overflow to inf, NaN kept. */
static uint16_t lg_f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf or nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? (0x200u | ((ax >> 13) & 0x3ffu)) : 0u));
    if (ax >= 0x477ff000u) /* rounds to >= 65520: overflow */
        return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) { /* below 2^-14: subnormal half (or zero) */
        /* value / 2^-24, rounded to nearest even integer */
        float a;
        memcpy(&a, &ax, 4);
        double q = (double)a * 16777216.0; /* exact */
        double r = nearbyint(q);            /* default rounding mode: to nearest even */
        return (uint16_t)(sign | (uint16_t)r);
    }
    uint32_t e = (ax >> 23) - 112; /* half exponent field, 1..30 */
    uint32_t m = ax & 0x7fffffu;
    uint32_t hm = m >> 13, rem = m & 0x1fffu;
    uint32_t h = (e << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) h += 1; /* carries into the exponent correctly */
    return (uint16_t)(sign | h);
}

static float sigmoid0(float a) { return (float)(1.0 / (1.0 + exp(-(double)a))); }
static float sigmoid1(float a) { return 1.0f / (1.0f + expf(-a)); }

/* Dot product of fp16 rows w and x over D (no bias), in `order`. */
static float lg_dot(const uint16_t* w, const uint16_t* x, int64_t D, int order, float init) {
    if (order == 1) {
        float acc = init;
        for (int64_t d = 0; d < D; ++d) acc = acc + lg_h2f(w[d]) * lg_h2f(x[d]);
        return acc;
    }
    float p[64];
    for (int l = 0; l < 64; ++l) p[l] = 0.0f;
    for (int64_t d = 0; d < D; ++d) {
        int l = (int)((d % 512) / 8);
        p[l] = p[l] + lg_h2f(w[d]) * lg_h2f(x[d]);
    }
    for (int s = 32; s >= 1; s >>= 1) {
        float q[64];
        for (int l = 0; l < 64; ++l) q[l] = p[l] + p[l ^ s];
        memcpy(p, q, sizeof(p));
    }
    return p[0] + init;
}

static float lg_bias(const uint16_t* b, int64_t n) { return b ? lg_h2f(b[n]) : 0.0f; }

ORACLE_API float oracle_lg_dot(const uint16_t* w, const uint16_t* x, int64_t D, int order) {
    return lg_dot(w, x, D, order, 0.0f);
}

ORACLE_API uint16_t oracle_lg_f2h(float f) { return lg_f2h(f); }

ORACLE_API void oracle_lg_predict(const uint16_t* x, const uint16_t* w, const uint16_t* bias, int64_t B,
                                  int64_t D, int64_t D_ffn, float threshold, int order, float* gate_out,
                                  uint8_t* mask, int32_t* idx, int32_t* count) {
    for (int64_t b = 0; b < B; ++b) {
        int32_t c = 0;
        for (int64_t n = 0; n < D_ffn; ++n) {
            float a = lg_dot(w + n * D, x + b * D, D, order, lg_bias(bias, n));
            float g = order == 1 ? sigmoid1(a) : sigmoid0(a);
            if (gate_out) gate_out[b * D_ffn + n] = g;
            uint8_t on = g >= threshold ? 1 : 0;
            mask[b * D_ffn + n] = on;
            if (on) idx[b * D_ffn + c++] = (int32_t)n;
        }
        count[b] = c;
    }
}

/* One SwiGLU value from the fp32 gate and up sums (sparse_matmul.cu:138-145):
 * both are stored as fp16 first, then silu(g) * u in fp32, stored as fp16. */
static uint16_t lg_swiglu(float g_acc, float u_acc, int order) {
    float g = lg_h2f(lg_f2h(g_acc)), u = lg_h2f(lg_f2h(u_acc));
    float s = order == 1 ? sigmoid1(g) : sigmoid0(g);
    float silu = g * s;
    return lg_f2h(silu * u);
}

/* Returns 0, or -1 when the sparse branch has no coverage (the reference's
 * launch would fail). */
ORACLE_API int oracle_lg_sparse_mlp(const uint16_t* x, const uint16_t* wg, const uint16_t* bg, const uint16_t* wu,
                                    const uint16_t* bu, const uint16_t* wd, const int32_t* idx,
                                    const int32_t* count, int64_t B, int64_t D, int64_t D_ffn,
                                    float sparsity_pct, int order, uint16_t* y) {
    float frac = sparsity_pct / 100.0f;
    int dense = frac < 0.30f;
    int64_t cover = D_ffn;
    if (!dense) {
        float m = (1.0f - frac) * (float)D_ffn;
        if (!(m > -256.0f)) return -1;
        int64_t max_active = (int64_t)m + 32;
        if (max_active > D_ffn) max_active = D_ffn;
        cover = max_active > 0 ? (max_active + 255) / 256 * 256 : 0;
        if (cover < 1) return -1;
    }
    uint16_t* act = (uint16_t*)calloc((size_t)(B * D_ffn), sizeof(uint16_t));
    int32_t* list = (int32_t*)malloc(sizeof(int32_t) * (size_t)D_ffn);
    int32_t* mult = (int32_t*)malloc(sizeof(int32_t) * (size_t)D_ffn);
    for (int64_t b = 0; b < B; ++b) {
        const uint16_t* xb = x + b * D;
        uint16_t* ab = act + b * D_ffn;
        int64_t lim;
        if (dense) {
            lim = D_ffn;
            for (int64_t i = 0; i < D_ffn; ++i) list[i] = (int32_t)i;
        } else {
            int64_t c = count[b];
            lim = c < 0 ? 0 : (c > D_ffn ? D_ffn : c);
            for (int64_t i = 0; i < lim; ++i) list[i] = idx[b * D_ffn + i];
        }
        int64_t gl = dense ? lim : (lim < cover ? lim : cover);
        for (int64_t i = 0; i < gl; ++i) {
            int64_t n = list[i];
            if (n < 0 || n >= D_ffn) continue;
            /* order 0 adds the bias after the tree, order 1 starts from it */
            float g = lg_dot(wg + n * D, xb, D, order, dense ? 0.0f : lg_bias(bg, n));
            float u = lg_dot(wu + n * D, xb, D, order, dense ? 0.0f : lg_bias(bu, n));
            ab[n] = lg_swiglu(g, u, order);
        }
        /* multiplicity of each neuron among the first lim list entries (the
         * dense branch lists every neuron once) */
        for (int64_t n = 0; n < D_ffn; ++n) mult[n] = 0;
        for (int64_t i = 0; i < lim; ++i) {
            int64_t n = list[i];
            if (n >= 0 && n < D_ffn) mult[n] += 1;
        }
        for (int64_t d = 0; d < D; ++d) {
            const uint16_t* wrow = wd + d * D_ffn;
            float out;
            if (order == 1) {
                float acc = 0.0f;
                for (int64_t i = 0; i < lim; ++i) {
                    int64_t n = list[i];
                    if (n < 0 || n >= D_ffn) continue;
                    acc = acc + lg_h2f(ab[n]) * lg_h2f(wrow[n]);
                }
                out = acc;
            } else {
                float p[64];
                for (int l = 0; l < 64; ++l) p[l] = 0.0f;
                for (int64_t n = 0; n < D_ffn; ++n) {
                    if (mult[n] == 0) continue;
                    int l = (int)((n % 512) / 8);
                    float a = (float)mult[n] * lg_h2f(ab[n]);
                    p[l] = fmaf(lg_h2f(wrow[n]), a, p[l]);
                }
                for (int s = 32; s >= 1; s >>= 1) {
                    float q[64];
                    for (int l = 0; l < 64; ++l) q[l] = p[l] + p[l ^ s];
                    memcpy(p, q, sizeof(p));
                }
                out = p[0];
            }
            y[b * D + d] = lg_f2h(out);
        }
    }
    free(mult);
    free(list);
    free(act);
    return 0;
}

ORACLE_API float oracle_lg_sparsity(const int32_t* count, int64_t B, int64_t D_ffn) {
    float total_active = 0.0f;
    for (int64_t b = 0; b < B; ++b) total_active += (float)count[b];
    float avg_active = total_active / (float)B;
    return (1.0f - avg_active / (float)D_ffn) * 100.0f;
}

/* ---------------------------------------------------------------------- */
/* oracle_lg_calibrate: kernels/sparse_moe/gate_calibrate.cu:54-85 (masks),
 * :105-210 (forward, gradient step), :228-340 (driver: zero start, `epochs`
 * full-batch steps at lr 1e-3, final forward, baseline sparsity and F1 on
 * the host).  order 0: this build's forward order (64 partials over
 * (d mod 512) / 8, fmaf, tree, then the bias) and fp64-based sigmoid;
 * order 1: the reference's loops (bias first, sequential fmaf) with this C
 * library's expf.  Both: gradients summed over samples in order with fmaf,
 * divided by N, applied as w = fmaf(-lr, g, w); predictions clamped to
 * [1e-7, 1 - 1e-7]. */
static float cal_dot0(const float* w, const float* x, int64_t D) {
    float p[64];
    for (int l = 0; l < 64; ++l) p[l] = 0.0f;
    for (int64_t d = 0; d < D; ++d) {
        int l = (int)((d % 512) / 8);
        p[l] = fmaf(w[d], x[d], p[l]);
    }
    for (int s = 32; s >= 1; s >>= 1) {
        float q[64];
        for (int l = 0; l < 64; ++l) q[l] = p[l] + p[l ^ s];
        memcpy(p, q, sizeof(p));
    }
    return p[0];
}

ORACLE_API void oracle_lg_calibrate(const float* x, const float* act, int64_t N, int64_t D, int64_t D_ffn, int order,
                                    int epochs, float* w, float* b, uint8_t* masks, float* pred, int* enabled,
                                    float* f1_out, float* sparsity_out) {
    const float lr = 1e-3f;
    long long active_total = 0;
    for (int64_t s = 0; s < N; ++s) {
        const float* row = act + s * D_ffn;
        float m = 0.0f;
        for (int64_t i = 0; i < D_ffn; ++i) m = fmaxf(m, fabsf(row[i]));
        m = fmaxf(m, 1e-10f);
        const float thr = 0.01f * m;
        for (int64_t i = 0; i < D_ffn; ++i) {
            masks[s * D_ffn + i] = fabsf(row[i]) >= thr ? 1 : 0;
            active_total += masks[s * D_ffn + i];
        }
    }
    *sparsity_out = (1.0f - (float)active_total / ((float)N * (float)D_ffn)) * 100.0f;
    for (int64_t i = 0; i < D_ffn * D; ++i) w[i] = 0.0f;
    for (int64_t n = 0; n < D_ffn; ++n) b[n] = 0.0f;
    for (int ep = 0; ep <= epochs; ++ep) {
        for (int64_t s = 0; s < N; ++s)
            for (int64_t n = 0; n < D_ffn; ++n) {
                const float* wr = w + n * D;
                const float* xs = x + s * D;
                float a, p;
                if (order == 1) {
                    a = b[n];
                    for (int64_t d = 0; d < D; ++d) a = fmaf(xs[d], wr[d], a);
                    p = 1.0f / (1.0f + expf(-a));
                } else {
                    a = cal_dot0(wr, xs, D) + b[n];
                    p = (float)(1.0 / (1.0 + exp(-(double)a)));
                }
                pred[s * D_ffn + n] = fmaxf(1e-7f, fminf(1.0f - 1e-7f, p));
            }
        if (ep == epochs) break; /* the final forward only */
        for (int64_t n = 0; n < D_ffn; ++n) {
            float gb = 0.0f;
            for (int64_t s = 0; s < N; ++s) gb += pred[s * D_ffn + n] - (float)masks[s * D_ffn + n];
            for (int64_t d = 0; d < D; ++d) {
                float gw = 0.0f;
                for (int64_t s = 0; s < N; ++s)
                    gw = fmaf(pred[s * D_ffn + n] - (float)masks[s * D_ffn + n], x[s * D + d], gw);
                w[n * D + d] = fmaf(-lr, gw / (float)N, w[n * D + d]);
            }
            b[n] = fmaf(-lr, gb / (float)N, b[n]);
        }
    }
    long long tp = 0, fp = 0, fn = 0;
    for (int64_t i = 0; i < N * D_ffn; ++i) {
        int pr = pred[i] >= 0.5f, ac = masks[i] > 0;
        if (pr && ac) ++tp;
        else if (pr && !ac) ++fp;
        else if (!pr && ac) ++fn;
    }
    float precision = (tp + fp > 0) ? (float)tp / (float)(tp + fp) : 0.0f;
    float recall = (tp + fn > 0) ? (float)tp / (float)(tp + fn) : 0.0f;
    float f1 = (precision + recall > 0) ? 2.0f * precision * recall / (precision + recall) : 0.0f;
    *f1_out = f1;
    *enabled = f1 >= 0.70f;
}
