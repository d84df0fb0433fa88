/*
 * moe_oracle.c -- CPU restatement of the PHANTOM sparse-MoE layer path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.  The product path (libphantom_moe.so) never calls it and
 * has no CPU fallback.
 *
 * What each function restates (reference paths are relative to the
 * reference repository root):
 *
 *   oracle_q4_0_dequant   python/phantom/loader/gguf_loader.py:362-381
 *                         (numpy Q4_0 branch; the fp32 values computed at
 *                         :376-378, before the storage cast to bf16 at :380)
 *                         and :588-596 (torch branch, same arithmetic).
 *   oracle_route          tests/test_moe_routing.py:56-72
 *                         (logits = x W^T, torch.topk largest/sorted, softmax
 *                         over the k selected logits), with the logit
 *                         arithmetic fixed by the numeric contract below, and
 *                         the sigmoid-renormalised variant used for the
 *                         DeepSeek-V3-style layer.
 *   oracle_permute        kernels/sparse_moe/gate_predict.cu:153-177 is the
 *                         reference's only compaction; the MoE permute is the
 *                         stable counting sort of (token, slot) pairs by
 *                         expert: offsets = exclusive_cumsum(bincount(idx)),
 *                         order = stable_argsort(idx.flatten()).
 *   oracle_expert_ffn     kernels/sparse_moe/sparse_matmul.cu:120-146 and
 *                         :187-215 (SwiGLU h = silu(g) * u, silu(g) =
 *                         g * 1/(1+exp(-g)); y = W_down h), evaluated in fp64
 *                         on exact fp32 dequantised weights.
 *   oracle_moe_forward    the whole layer: route -> experts -> weighted
 *                         combine y[t] = sum_j w[t,j] * FFN_{e[t,j]}(x[t]) in
 *                         slot order j = 0..k-1, plus the always-on shared
 *                         expert with weight 1.0 when present (the combine has
 *                         no reference code; its semantics are the
 *                         index_add_ of w*y that transformers' MoE blocks do,
 *                         which is what python/phantom/phantom_cli.py:1393-1430
 *                         runs).
 *
 * Numeric contract for router logits (shared with the HIP router kernel so
 * that expert selection is bit-exact):
 *   - x (bf16 or fp32) and W (fp32) are widened to fp64; each product x*w is
 *     exact in fp64 (at most 24+24 significant bits).
 *   - 64 partial sums: partial l accumulates, in increasing h, the products
 *     for every h with (h mod 256) / 4 == l, starting from +0.0.
 *   - The partials are combined by the pairwise tree
 *       p[l] <- p[l] + p[l xor s]  for s = 32, 16, 8, 4, 2, 1
 *     and the logit is p[0].  The router bias (if any) is then added in fp64.
 *   - Selection: the k largest logits, sorted descending; equal logits are
 *     ordered by the lower expert index first.  NaN logits rank below every
 *     number (they are never preferred over a finite logit).
 *   - Weights (fp32): softmax over the k selected logits (score mode 0), or
 *     sigmoid(l_j) / sum_i sigmoid(l_i) over the k selected (score mode 1),
 *     computed in fp64 then rounded to fp32.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------ */
/* scalar conversions                                                 */
/* ------------------------------------------------------------------ */

/* IEEE binary16 -> binary32, exact (normals, subnormals, inf, nan). */
static float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* subnormal: value = man * 2^-24 */
            float v = (float)man * (1.0f / 16777216.0f);
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static float bf16_to_float(uint16_t b) {
    uint32_t bits = (uint32_t)b << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

ORACLE_API float oracle_half_to_float(uint16_t h) { return half_to_float(h); }

/* ------------------------------------------------------------------ */
/* Q4_0 dequantisation                                                 */
/* ------------------------------------------------------------------ */

/* One Q4_0 block: 18 bytes = fp16 d (little endian) + 16 bytes qs.
 * Element j (0..15)  = ((qs[j] & 0xF) - 8) * d
 * Element j+16       = ((qs[j] >> 4)  - 8) * d
 * (gguf_loader.py:369-378).  The product of a 4-bit integer and an fp16
 * scale is exact in fp32. */
ORACLE_API void oracle_q4_0_dequant(const uint8_t* blocks, int64_t n_blocks, float* out) {
#pragma omp parallel for schedule(static) if (n_blocks > 65536)
    for (int64_t b = 0; b < n_blocks; ++b) {
        const uint8_t* blk = blocks + b * 18;
        float d = half_to_float((uint16_t)(blk[0] | (blk[1] << 8)));
        const uint8_t* qs = blk + 2;
        float* o = out + b * 32;
        for (int j = 0; j < 16; ++j) {
            int lo = (int)(qs[j] & 0x0f) - 8;
            int hi = (int)((qs[j] >> 4) & 0x0f) - 8;
            o[j] = (float)lo * d;
            o[j + 16] = (float)hi * d;
        }
    }
}

/* ------------------------------------------------------------------ */
/* Router                                                              */
/* ------------------------------------------------------------------ */

/* The fixed-order fp64 dot product of the numeric contract above. */
ORACLE_API double oracle_canonical_dot(const float* x, const float* w, int64_t H) {
    double p[64];
    double q[64];
    for (int l = 0; l < 64; ++l) p[l] = 0.0;
    for (int64_t h = 0; h < H; ++h) {
        int l = (int)((h & 255) >> 2);
        double prod = (double)x[h] * (double)w[h]; /* exact */
        p[l] = p[l] + prod;
    }
    for (int s = 32; s >= 1; s >>= 1) {
        for (int l = 0; l < 64; ++l) q[l] = p[l] + p[l ^ s];
        for (int l = 0; l < 64; ++l) p[l] = q[l];
    }
    return p[0];
}

/* a ranks strictly before b (value descending, index ascending, NaN last). */
static int ranks_before(double va, int ia, double vb, int ib) {
    int na = isnan(va), nb = isnan(vb);
    if (na || nb) {
        if (na && nb) return ia < ib;
        return nb; /* a is a number, b is NaN */
    }
    if (va > vb) return 1;
    if (va < vb) return 0;
    return ia < ib;
}

/* Select the k best of E logits in rank order. */
static void select_topk(const double* logits, int E, int k, int32_t* idx_out, double* val_out) {
    unsigned char* taken = (unsigned char*)calloc((size_t)E, 1);
    for (int j = 0; j < k; ++j) {
        int best = -1;
        for (int e = 0; e < E; ++e) {
            if (taken[e]) continue;
            if (best < 0 || ranks_before(logits[e], e, logits[best], best)) best = e;
        }
        taken[best] = 1;
        idx_out[j] = best;
        val_out[j] = logits[best];
    }
    free(taken);
}

/* Weights over the selected logits (score_mode 0: softmax, 1: sigmoid renorm). */
static void topk_weights(const double* v, int k, int score_mode, float* w_out) {
    double e[256];
    double s = 0.0;
    if (score_mode == 0) {
        double m = v[0];
        for (int j = 0; j < k; ++j) {
            e[j] = exp(v[j] - m);
            s += e[j];
        }
    } else {
        for (int j = 0; j < k; ++j) {
            e[j] = 1.0 / (1.0 + exp(-v[j]));
            s += e[j];
        }
    }
    for (int j = 0; j < k; ++j) w_out[j] = (float)(e[j] / s);
}

/*
 * Route T tokens.  x: [T,H] as fp32 values (bf16 inputs are widened exactly
 * by the caller); W: [E,H] fp32 (nn.Linear weight layout); bias: [E] or NULL.
 * Outputs: idx [T,k] int32, w [T,k] fp32, logits [T,E] fp64 (may be NULL).
 */
ORACLE_API int oracle_route(const float* x, const float* W, const float* bias, int64_t T, int64_t H,
                            int E, int k, int score_mode, int32_t* idx, float* w, double* logits_out) {
    if (k < 1 || k > E || k > 256 || E < 1) return -1;
    double* lg = (double*)malloc(sizeof(double) * (size_t)E);
    double vals[256];
    for (int64_t t = 0; t < T; ++t) {
        for (int e = 0; e < E; ++e) {
            double v = oracle_canonical_dot(x + t * H, W + (int64_t)e * H, H);
            if (bias) v = v + (double)bias[e];
            lg[e] = v;
            if (logits_out) logits_out[t * E + e] = v;
        }
        select_topk(lg, E, k, idx + t * k, vals);
        topk_weights(vals, k, score_mode, w + t * k);
    }
    free(lg);
    return 0;
}

/* ------------------------------------------------------------------ */
/* Permute (stable counting sort by expert)                            */
/* ------------------------------------------------------------------ */

/* idx: [n_slots] expert ids (slot s = t*k + j).  Outputs:
 *   offsets[E+1]      exclusive prefix sum of per-expert counts
 *   sorted_slots[n]   slots ordered by (expert, slot)
 *   slot_pos[n]       inverse: position of slot s in sorted order */
ORACLE_API int oracle_permute(const int32_t* idx, int64_t n_slots, int E, int32_t* offsets,
                              int32_t* sorted_slots, int32_t* slot_pos) {
    int64_t* cursor = (int64_t*)calloc((size_t)E + 1, sizeof(int64_t));
    for (int64_t s = 0; s < n_slots; ++s) {
        if (idx[s] < 0 || idx[s] >= E) {
            free(cursor);
            return -1;
        }
        cursor[idx[s] + 1] += 1;
    }
    for (int e = 0; e < E; ++e) cursor[e + 1] += cursor[e];
    for (int e = 0; e <= E; ++e) offsets[e] = (int32_t)cursor[e];
    for (int64_t s = 0; s < n_slots; ++s) {
        int64_t p = cursor[idx[s]]++;
        sorted_slots[p] = (int32_t)s;
        slot_pos[s] = (int32_t)p;
    }
    free(cursor);
    return 0;
}

/* ------------------------------------------------------------------ */
/* Expert FFN (fp64)                                                   */
/* ------------------------------------------------------------------ */

/* SwiGLU expert on dequantised fp32 weights, fp64 arithmetic.
 *   wg, wu: [I,H]; wd: [H,I]; x: [H]; y: [H] (fp64 out).
 * g = wg x, u = wu x, h = silu(g) * u, y = wd h. */
static void expert_ffn_f64(const float* x, const float* wg, const float* wu, const float* wd, int64_t H,
                           int64_t I, double* hbuf, double* y) {
    /* Rows are independent and each dot product is sequential, so the
     * row-parallel loops give the same bits for any thread count. */
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < I; ++i) {
        const float* rg = wg + i * H;
        const float* ru = wu + i * H;
        double g = 0.0, u = 0.0;
        for (int64_t c = 0; c < H; ++c) {
            g += (double)rg[c] * (double)x[c];
            u += (double)ru[c] * (double)x[c];
        }
        double silu = g * (1.0 / (1.0 + exp(-g)));
        hbuf[i] = silu * u;
    }
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < H; ++r) {
        const float* rd = wd + r * I;
        double acc = 0.0;
        for (int64_t i = 0; i < I; ++i) acc += (double)rd[i] * hbuf[i];
        y[r] = acc;
    }
}

/* One expert on Q4_0 bytes: gate/up [I, H/32 blocks], down [H, I/32 blocks]. */
ORACLE_API int oracle_expert_ffn(const float* x, const uint8_t* gate_q4, const uint8_t* up_q4,
                                 const uint8_t* down_q4, int64_t H, int64_t I, double* y) {
    if (H % 32 || I % 32) return -1;
    float* wg = (float*)malloc(sizeof(float) * (size_t)(I * H));
    float* wu = (float*)malloc(sizeof(float) * (size_t)(I * H));
    float* wd = (float*)malloc(sizeof(float) * (size_t)(I * H));
    double* hb = (double*)malloc(sizeof(double) * (size_t)I);
    oracle_q4_0_dequant(gate_q4, I * H / 32, wg);
    oracle_q4_0_dequant(up_q4, I * H / 32, wu);
    oracle_q4_0_dequant(down_q4, I * H / 32, wd);
    expert_ffn_f64(x, wg, wu, wd, H, I, hb, y);
    free(wg);
    free(wu);
    free(wd);
    free(hb);
    return 0;
}

/* ------------------------------------------------------------------ */
/* Whole layer                                                         */
/* ------------------------------------------------------------------ */

/*
 * x: [n, H] fp32 (the tokens to evaluate; bf16 inputs widened exactly).
 * router_w: [E, H] fp32; router_bias: [E] or NULL.
 * gate_q4/up_q4: [E][I][H/32][18]; down_q4: [E][H][I/32][18].
 * sh_*: shared expert (same shapes, one expert) or NULL.
 * Outputs: y [n, H] fp32, idx [n, k], w [n, k].
 *
 * Experts are visited in ascending id; each needed expert is dequantised
 * once.  Per-slot expert outputs are kept in fp64 and combined in slot order.
 */
ORACLE_API int oracle_moe_forward(const float* x, int64_t n, int64_t H, int64_t I, int E, int k,
                                  int score_mode, const float* router_w, const float* router_bias,
                                  const uint8_t* gate_q4, const uint8_t* up_q4, const uint8_t* down_q4,
                                  const uint8_t* sh_gate, const uint8_t* sh_up, const uint8_t* sh_down,
                                  float* y, int32_t* idx, float* w) {
    if (H % 32 || I % 32 || k < 1 || k > E) return -1;
    int rc = oracle_route(x, router_w, router_bias, n, H, E, k, score_mode, idx, w, NULL);
    if (rc) return rc;

    const int64_t gu_bytes = I * (H / 32) * 18;
    const int64_t dn_bytes = H * (I / 32) * 18;
    double* ye = (double*)calloc((size_t)(n * k * H), sizeof(double));
    double* ysh = NULL;
    float* wg = (float*)malloc(sizeof(float) * (size_t)(I * H));
    float* wu = (float*)malloc(sizeof(float) * (size_t)(I * H));
    float* wd = (float*)malloc(sizeof(float) * (size_t)(I * H));
    double* hb = (double*)malloc(sizeof(double) * (size_t)I);
    if (!ye || !wg || !wu || !wd || !hb) return -2;

    for (int e = 0; e < E; ++e) {
        int used = 0;
        for (int64_t s = 0; s < n * k; ++s) used |= (idx[s] == e);
        if (!used) continue;
        oracle_q4_0_dequant(gate_q4 + e * gu_bytes, I * H / 32, wg);
        oracle_q4_0_dequant(up_q4 + e * gu_bytes, I * H / 32, wu);
        oracle_q4_0_dequant(down_q4 + e * dn_bytes, I * H / 32, wd);
        for (int64_t s = 0; s < n * k; ++s) {
            if (idx[s] != e) continue;
            expert_ffn_f64(x + (s / k) * H, wg, wu, wd, H, I, hb, ye + s * H);
        }
    }
    if (sh_gate && sh_up && sh_down) {
        ysh = (double*)calloc((size_t)(n * H), sizeof(double));
        oracle_q4_0_dequant(sh_gate, I * H / 32, wg);
        oracle_q4_0_dequant(sh_up, I * H / 32, wu);
        oracle_q4_0_dequant(sh_down, I * H / 32, wd);
        for (int64_t t = 0; t < n; ++t) expert_ffn_f64(x + t * H, wg, wu, wd, H, I, hb, ysh + t * H);
    }
    for (int64_t t = 0; t < n; ++t) {
        for (int64_t r = 0; r < H; ++r) {
            double acc = 0.0;
            for (int j = 0; j < k; ++j) acc += (double)w[t * k + j] * ye[(t * k + j) * H + r];
            if (ysh) acc += ysh[t * H + r];
            y[t * H + r] = (float)acc;
        }
    }
    free(ye);
    free(ysh);
    free(hb);
    free(wg);
    free(wu);
    free(wd);
    return 0;
}

/* bf16 -> fp32 widening helper for callers holding raw bf16 bits. */
ORACLE_API void oracle_bf16_to_float(const uint16_t* in, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = bf16_to_float(in[i]);
}
