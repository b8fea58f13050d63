/*
 * lro_int8.c -- the CPU oracle for MiniMax H3's INT8 attention chain (quantised Q, K, V; softmax(QK^T/sqrt(128)) V).
 *
 * TEST INFRASTRUCTURE ONLY, like lro.c: only tests/ and __graft_entry__.smoke() load it, as the checker.
 *
 * What it restates (reference = jayleaton/localrouter, read-only; the kernels are comfy-kitchen v0.2.35's
 * SageAttention INT8 path, vendored at kernels/cuda/minimax/kitchen/ and launched by
 * src/engines/minimax_h3/launch.zig:317-419):
 *   - the K anchor (detect_k_anchor, quant_qk_int8.cu:461-596): nine evenly spaced sample keys per head; the sample
 *     closest to the others becomes the anchor subtracted from every key when that lowers the samples' energy without
 *     raising their abs-max by more than 12.5 %. Subtracting one key from all keys shifts every score of a query by
 *     the same amount, so softmax is unchanged;
 *   - the Hadamard rotations applied to Q and K before quantisation (quant_qk_int8.cu:75-155), in the same
 *     operation order: H4 on each lane's 4 channels; or, for head dim 128, a fixed sign flip followed by the
 *     normalised H128 built as H4 within a lane and five xor butterflies across 32 lanes (channel 4l + c belongs to
 *     lane l); or, for head dim 64, the plain normalised H64: H4 within a lane and four xor butterflies across 16
 *     lanes, times 1/4 (convrot64). Q and K get the same orthogonal rotation, so their dot products are unchanged;
 *   - int8 quantisation by round-to-nearest-even with saturation of x * (1 / scale) (float_utils.cuh:40-51), with
 *     scale = absmax / 127 + 1e-7 for Q and K (quant_qk_int8.cu:245-247) and max(absmax / 127, 1e-12) per channel for
 *     V (quant_v_int8.cu:113-116);
 *   - the attention over the quantised operands: s = (q8 . k8) * q_scale * k_scale * scale (the caller's scale: H3
 *     passes 128^-0.5 as fp32, 0x3DB504F3, launch.zig:414), softmax over all keys, O = sum_j P_j (v8_j * v_scale).
 * Head dims 128 (the engine's) and 64 (the wheel's other case, kitchen_launch.cu:196-241); d is an argument.
 * Scale granularity is this build's choice (one Q scale per query row, one K scale per 16 consecutive keys, one V
 * scale per channel), not the reference's thread-group layout; the arithmetic inside a group is the reference's.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define DMAX 128

static float bf16f(uint16_t h) {
    union { uint32_t u; float f; } v;
    v.u = (uint32_t)h << 16;
    return v.f;
}

static float flip_sign(float x, uint32_t flip) {
    union { uint32_t u; float f; } v;
    v.f = x;
    v.u ^= flip << 31;
    return v.f;
}

/* round to nearest even, saturated to [-128, 127] */
static int8_t rn_sat_s8(float x) {
    if (x != x) return 0;
    const float r = rintf(x);   /* default rounding mode: nearest even */
    if (r >= 127.0f) return 127;
    if (r <= -128.0f) return -128;
    return (int8_t)r;
}

static void convrot4(float* v) {
    const float x0 = v[0], x1 = v[1], x2 = v[2], x3 = v[3];
    const float a0 = x0 + x1, a1 = x0 - x1, a2 = x2 + x3, a3 = x2 - x3;
    v[0] = (a0 + a2) * 0.5f;
    v[1] = (a1 + a3) * 0.5f;
    v[2] = (a0 - a2) * 0.5f;
    v[3] = (a1 - a3) * 0.5f;
}

/* One row of d channels (d / 4 lanes of 4). kind 0: none; 4: H4 per lane; 128: sign flip + H128 (d 128);
 * 64: H64 (d 64). */
void lro_i8_rotate(float* x, int d, int kind) {
    if (kind == 0) return;
    const int lanes = d / 4;
    if (kind == 128) {
        static const uint32_t signs[4] = {0x1035997bu, 0x8087f5eeu, 0xee2e4e1au, 0x71132418u};
        for (int lane = 0; lane < 32; ++lane) {
            const uint32_t s = signs[lane >> 3];
            const int shift = (lane & 7) * 4;
            for (int c = 0; c < 4; ++c) x[4 * lane + c] = flip_sign(x[4 * lane + c], ((s >> (shift + c)) & 1u) ^ 1u);
        }
    }
    for (int lane = 0; lane < lanes; ++lane) convrot4(x + 4 * lane);
    if (kind != 128 && kind != 64) return;
    float prev[DMAX];
    for (int bit = 1; bit < lanes; bit <<= 1) {
        memcpy(prev, x, sizeof(float) * (size_t)d);
        for (int lane = 0; lane < lanes; ++lane)
            for (int c = 0; c < 4; ++c) {
                const float mine = prev[4 * lane + c], other = prev[4 * (lane ^ bit) + c];
                x[4 * lane + c] = (lane & bit) ? other - mine : mine + other;
            }
    }
    const float norm = kind == 128 ? 0.1767766952966369f : 0.25f;
    for (int i = 0; i < d; ++i) x[i] *= norm;
}

/* One kv head's anchor row, or -1. k: the head's first key, rows k_rs elements apart, Lk keys of d channels. */
int lro_i8_anchor(const uint16_t* k, int64_t k_rs, int Lk, int d) {
    enum { NS = 9 };
    double s[NS][DMAX];
    for (int i = 0; i < NS; ++i) {
        const int row = (int)((int64_t)i * (Lk - 1) / (NS - 1));
        for (int c = 0; c < d; ++c) s[i][c] = bf16f(k[(int64_t)row * k_rs + c]);
    }
    double orig_e = 0.0, orig_m = 0.0, dist[NS] = {0};
    for (int c = 0; c < d; ++c) {
        double sum = 0.0;
        for (int i = 0; i < NS; ++i) {
            orig_e += s[i][c] * s[i][c];
            orig_m = fmax(orig_m, fabs(s[i][c]));
            sum += s[i][c];
        }
        for (int j = 0; j < NS; ++j) {
            const double d = NS * s[j][c] - sum;
            dist[j] += d * d;
        }
    }
    int best = 0;
    for (int j = 1; j < NS; ++j)
        if (dist[j] < dist[best]) best = j;
    double best_e = 0.0, best_m = 0.0;
    for (int c = 0; c < d; ++c)
        for (int i = 0; i < NS; ++i) {
            const double r = s[i][c] - s[best][c];
            best_e += r * r;
            best_m = fmax(best_m, fabs(r));
        }
    const int improves = best_e < orig_e && best_m <= orig_m * 1.125;
    return improves ? (int)((int64_t)best * (Lk - 1) / (NS - 1)) : -1;
}

/* Quantise `rows` rows of one head (d channels): subtract row `anchor` (>= 0) first, rotate, then one scale per
 * `group` rows (group 1: per row). out: int8 [rows][d]; scales: [ceil(rows / group)]. */
void lro_i8_quant_rows(const uint16_t* x, int64_t x_rs, int rows, int d, int rot, int anchor, int group, int8_t* out,
                       float* scales) {
    float a[DMAX];
    for (int c = 0; c < d; ++c) a[c] = anchor >= 0 ? bf16f(x[(int64_t)anchor * x_rs + c]) : 0.0f;
    for (int g0 = 0; g0 < rows; g0 += group) {
        const int n = rows - g0 < group ? rows - g0 : group;
        float v[64][DMAX];   /* group <= 64 */
        float mx = 0.0f;
        for (int r = 0; r < n; ++r) {
            for (int c = 0; c < d; ++c) v[r][c] = bf16f(x[(int64_t)(g0 + r) * x_rs + c]) - a[c];
            lro_i8_rotate(v[r], d, rot);
            for (int c = 0; c < d; ++c) mx = fmaxf(mx, fabsf(v[r][c]));
        }
        const float sc = mx / 127.0f + 1e-7f;
        const float inv = 1.0f / sc;
        scales[g0 / group] = sc;
        for (int r = 0; r < n; ++r)
            for (int c = 0; c < d; ++c) out[(int64_t)(g0 + r) * d + c] = rn_sat_s8(v[r][c] * inv);
    }
}

/* V of one head: one scale per channel over all rows. out: int8 [rows][d]; scales: [d]. */
void lro_i8_quant_v(const uint16_t* v, int64_t v_rs, int rows, int d, int8_t* out, float* scales) {
    for (int c = 0; c < d; ++c) {
        float mx = 0.0f;
        for (int r = 0; r < rows; ++r) mx = fmaxf(mx, fabsf(bf16f(v[(int64_t)r * v_rs + c])));
        const float sc = fmaxf(mx * (1.0f / 127.0f), 1e-12f);
        const float inv = 1.0f / sc;
        scales[c] = sc;
        for (int r = 0; r < rows; ++r) out[(int64_t)r * d + c] = rn_sat_s8(bf16f(v[(int64_t)r * v_rs + c]) * inv);
    }
}

/* Attention of one head over its quantised operands, fp64: q8 [W][d] with qs [W] (one per row); k8 [nk][d] with
 * ks [ceil(nk / kgroup)]; v8 [nk][d] with vs [d]; out fp32 [W][d]; scale the softmax scale (fp32). */
void lro_i8_attention(const int8_t* q8, const float* qs, const int8_t* k8, const float* ks, int kgroup,
                      const int8_t* v8, const float* vs, int W, int nk, int d, float scale, float* out) {
    const int D = d;
#pragma omp parallel
    {
    double* s = (double*)malloc(sizeof(double) * (size_t)nk);
#pragma omp for schedule(dynamic, 4)
    for (int i = 0; i < W; ++i) {
        double m = -INFINITY;
        for (int j = 0; j < nk; ++j) {
            int64_t dot = 0;
            for (int c = 0; c < D; ++c) dot += (int64_t)q8[(int64_t)i * D + c] * k8[(int64_t)j * D + c];
            s[j] = (double)dot * qs[i] * ks[j / kgroup] * (double)scale;
            if (s[j] > m) m = s[j];
        }
        double l = 0.0, o[DMAX] = {0};
        for (int j = 0; j < nk; ++j) {
            const double p = exp(s[j] - m);
            l += p;
            for (int c = 0; c < D; ++c) o[c] += p * v8[(int64_t)j * D + c];
        }
        for (int c = 0; c < D; ++c) out[(int64_t)i * D + c] = (float)(o[c] / l * vs[c]);
    }
    free(s);
    }
}

/* The same attention with P rounded the way the reference's kernel rounds it (attn_utils.cuh:610-695): per key tile of
 * `cta` keys (tiles start at multiples of cta) and per query row, m_t = max_j x_j - 7.9943534 with x_j = s_j * log2(e);
 * P_j = round(exp2(x_j - m_t)) in [0, 255]; the row sum is taken over the rounded P; tile t enters O and the row sum
 * with weight exp2(m_t - M), M = max_t m_t. fp64 otherwise. */
void lro_i8_attention_p8(const int8_t* q8, const float* qs, const int8_t* k8, const float* ks, int kgroup,
                         const int8_t* v8, const float* vs, int W, int nk, int d, float scale, int cta, float* out) {
    const int D = d;
    const double log2e = 1.4426950408889634, offset = (double)7.9943534f;
    const int ntiles = (nk + cta - 1) / cta;
#pragma omp parallel
    {
    double* x = (double*)malloc(sizeof(double) * (size_t)nk);
    double* mt = (double*)malloc(sizeof(double) * (size_t)ntiles);
#pragma omp for schedule(dynamic, 4)
    for (int i = 0; i < W; ++i) {
        for (int j = 0; j < nk; ++j) {
            int64_t dot = 0;
            for (int c = 0; c < D; ++c) dot += (int64_t)q8[(int64_t)i * D + c] * k8[(int64_t)j * D + c];
            x[j] = (double)dot * qs[i] * ks[j / kgroup] * (double)scale * log2e;
        }
        double M = -INFINITY;
        for (int t = 0; t < ntiles; ++t) {
            double m = -INFINITY;
            for (int j = t * cta; j < nk && j < (t + 1) * cta; ++j) m = x[j] > m ? x[j] : m;
            mt[t] = m - offset;
            if (mt[t] > M) M = mt[t];
        }
        double l = 0.0, o[DMAX] = {0};
        for (int t = 0; t < ntiles; ++t) {
            const double w = exp2(mt[t] - M);
            double lt = 0.0, ot[DMAX] = {0};
            for (int j = t * cta; j < nk && j < (t + 1) * cta; ++j) {
                double p = rint(exp2(x[j] - mt[t]));
                p = p < 0.0 ? 0.0 : p > 255.0 ? 255.0 : p;
                lt += p;
                for (int c = 0; c < D; ++c) ot[c] += p * v8[(int64_t)j * D + c];
            }
            l += w * lt;
            for (int c = 0; c < D; ++c) o[c] += w * ot[c];
        }
        for (int c = 0; c < D; ++c) out[(int64_t)i * D + c] = (float)(o[c] / l * vs[c]);
    }
    free(x);
    free(mt);
    }
}
