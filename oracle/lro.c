/*
 * lro.c -- the CPU oracle for the DiT joint-attention path (QK-RMSNorm + RoPE + non-causal/causal attention).
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker or as the reported CPU baseline. The product path (localrouter_amd) never calls it.
 *
 * What it restates (reference = jayleaton/localrouter, read-only):
 *   - attention: kernels/cuda/qwen_image/attention.cu:253-444 (pattn2_kernel) and its launcher
 *     src/engines/qwen_image/ops_launch.zig:163-172. O_i = softmax_j(scale * <q_i, k_j>) v_j over keys j < nkeys,
 *     and j <= p0 + i when causal (attention.cu:304 `vis`); query head h reads kv head h / (H / HK)
 *     (attention.cu:264-266); keys past nkeys never contribute (attention.cu:275-276, zero-filled and masked).
 *   - per-head RMSNorm + RoPE: kernels/cuda/minimax/kitchen/rms_rope.cu:37-230 with rope_device.cuh:65-98
 *     (rrms = 1/sqrt(sum(x^2)/D + eps), y = x * rrms * w, pairs rotated by a 2x2 matrix [f00 f01; f10 f11],
 *     split-half pairs (i, i + rot/2), dims >= rot norm-only), and the Qwen-Image form
 *     src/engines/qwen_image/triton_k.zig:44-53 + tools/twin/stk_twin/dit.py:225-233 (fp32 weight, fp32 cos/sin
 *     [N, rot/2]); the interleaved pairing (2p, 2p+1) follows kernels/cuda/kandinsky6/dit/ops.cu:197-235.
 *     By default the oracle keeps the normalised value in full precision; with round_norm it rounds it to bf16
 *     before the rotation, as rms_rope.cu:143-150 does (the MiniMax H3 path).
 *
 * Two attention implementations:
 *   lro_attention_f64  -- brute force, double accumulation, two passes per row. This is the pin.
 *   lro_attention_f32  -- fp32, flash-style blocked (32 queries x 64 keys), online softmax, OpenMP over
 *                         (head, query block). This is the CPU baseline that bench.py times; it is checked
 *                         against lro_attention_f64 in tests/.
 *
 * Every function is pinned by tests/test_oracle.py (closed forms, invariants, torch-CPU SDPA, fp64 numpy brute
 * force, the reference's own RoPE-id vectors) and by planted mistakes (lro_set_mutant) that those pins must catch.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define LRO_D 128

/* Planted mistakes, used only by tests to show that the pins catch them (0 = none). */
enum {
    MUT_NONE = 0,
    MUT_ROPE_SIGN = 1,     /* y0 = c*x0 + s*x1 instead of c*x0 - s*x1 */
    MUT_NO_EPS = 2,        /* eps dropped from the RMS */
    MUT_PAIRING = 3,       /* interleaved <-> split-half swapped */
    MUT_NO_SCALE = 4,      /* scale not applied */
    MUT_CAUSAL_OFF1 = 5,   /* causal mask j < p0 + i instead of j <= p0 + i */
    MUT_GQA_MOD = 6,       /* kv head h % HK instead of h / (H / HK) */
    MUT_NO_WEIGHT = 7,     /* norm weight ignored */
    MUT_TABLE_T = 8,       /* 2x2 rotation matrix transposed */
    MUT_NO_ROUND = 9,      /* round_norm ignored: the normalised value kept unrounded before the rotation */
    MUT_NO_ROUND_PREP = 10, /* round_prepared ignored: the joint attention's prepared q / k kept unrounded */
};
static int g_mutant = 0;
void lro_set_mutant(int m) { g_mutant = m; }
int lro_get_mutant(void) { return g_mutant; }

int lro_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void lro_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* ---------------------------------------------------------------- bf16 <-> f32 (round to nearest even) */
float lro_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t lro_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40); /* quiet NaN */
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

void lro_f32_to_bf16_array(const float* x, uint16_t* y, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) y[i] = lro_f32_to_bf16(x[i]);
}

void lro_bf16_to_f32_array(const uint16_t* x, float* y, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) y[i] = lro_bf16_to_f32(x[i]);
}

/* ---------------------------------------------------------------- seeded N(0,1) bf16 inputs
 * Counter-based: key = mix(seed * 0x9E3779B97F4A7C15 + stream); for pair p, a = mix(key + 2p), b = mix(key + 2p + 1),
 * u1 = ((a >> 11) + 1) * 2^-53 in (0, 1], u2 = (b >> 11) * 2^-53, r = sqrt(-2 ln u1),
 * x[2p] = r cos(2 pi u2), x[2p + 1] = r sin(2 pi u2), each rounded to bf16 (RNE). mix is splitmix64's finaliser. */
static inline uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void lro_synth_normal_bf16(uint64_t seed, uint64_t stream, int64_t n, uint16_t* out) {
    const uint64_t key = mix64(seed * 0x9E3779B97F4A7C15ull + stream);
    const int64_t pairs = (n + 1) / 2;
    const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < pairs; ++p) {
        const uint64_t a = mix64(key + 2 * (uint64_t)p), b = mix64(key + 2 * (uint64_t)p + 1);
        const double u1 = ((double)(a >> 11) + 1.0) * 0x1.0p-53, u2 = (double)(b >> 11) * 0x1.0p-53;
        const double r = sqrt(-2.0 * log(u1));
        out[2 * p] = lro_f32_to_bf16((float)(r * cos(two_pi * u2)));
        if (2 * p + 1 < n) out[2 * p + 1] = lro_f32_to_bf16((float)(r * sin(two_pi * u2)));
    }
}

/* ---------------------------------------------------------------- RMSNorm + RoPE
 * table_kind: 0 = none (norm only), 1 = cos/sin fp32 [rows][rot/2] in ta (cos) and tb (sin) with row stride
 *             tab_stride (elements), 2 = 2x2 bf16 [rows][rot/2][2][2] in ta with row stride tab_stride (elements),
 *             3 = 2x2 fp32, same layout as 2.
 * pairing: 0 = interleaved (2p, 2p+1), 1 = split-half (p, p + rot/2).
 * w: fp32 [128] or NULL (ones); w_bf16: bf16 [128] used when w is NULL and w_bf16 is not.
 * x: bf16 [rows][heads][128] with row stride x_rs (elements, head h at h*128); y: fp32 [rows][heads][128] dense.
 * Row r uses table row r. (rms_rope.cu:83 rrms, :140-141 pairs, :161-164 rotation, :208-228 tail.)
 * round_norm != 0: the normalised, weighted value is rounded to fp32 and then to bf16 (RNE) before the rotation
 * (rms_rope.cu:143-150 stores x * rrms * w into a bf16 register pair before rotate_pair reads it). */
void lro_rms_rope_ex(const uint16_t* x, int64_t rows, int heads, int64_t x_rs, const float* w, const uint16_t* w_bf16,
                     int table_kind, const void* ta, const void* tb, int64_t tab_stride, int pairing, int rot,
                     float eps, int round_norm, float* y) {
    if (g_mutant == MUT_NO_ROUND) round_norm = 0;
    int pair_mode = pairing;
    if (g_mutant == MUT_PAIRING) pair_mode = 1 - pairing;
#pragma omp parallel for schedule(static)
    for (int64_t rh = 0; rh < rows * heads; ++rh) {
        const int64_t r = rh / heads;
        const int h = (int)(rh % heads);
        const uint16_t* xr = x + r * x_rs + (int64_t)h * LRO_D;
        float* yr = y + rh * LRO_D;
        double xs[LRO_D], ss = 0.0;
        for (int d = 0; d < LRO_D; ++d) {
            xs[d] = lro_bf16_to_f32(xr[d]);
            ss += xs[d] * xs[d];
        }
        const double e = g_mutant == MUT_NO_EPS ? 0.0 : (double)eps;
        const double rr = 1.0 / sqrt(ss / LRO_D + e);
        double n[LRO_D];
        for (int d = 0; d < LRO_D; ++d) {
            double wd = w ? (double)w[d] : (w_bf16 ? (double)lro_bf16_to_f32(w_bf16[d]) : 1.0);
            if (g_mutant == MUT_NO_WEIGHT) wd = 1.0;
            n[d] = xs[d] * rr * wd;
            if (round_norm) n[d] = lro_bf16_to_f32(lro_f32_to_bf16((float)n[d]));
        }
        if (table_kind != 0) {
            const int P = rot / 2;
            for (int p = 0; p < P; ++p) {
                const int a = pair_mode == 0 ? 2 * p : p, b = pair_mode == 0 ? 2 * p + 1 : p + P;
                double f00, f01, f10, f11;
                if (table_kind == 1) {
                    const double c = ((const float*)ta)[r * tab_stride + p], s = ((const float*)tb)[r * tab_stride + p];
                    f00 = c; f01 = -s; f10 = s; f11 = c;
                } else if (table_kind == 2) {
                    const uint16_t* m = (const uint16_t*)ta + r * tab_stride + 4 * p;
                    f00 = lro_bf16_to_f32(m[0]); f01 = lro_bf16_to_f32(m[1]);
                    f10 = lro_bf16_to_f32(m[2]); f11 = lro_bf16_to_f32(m[3]);
                } else {
                    const float* m = (const float*)ta + r * tab_stride + 4 * p;
                    f00 = m[0]; f01 = m[1]; f10 = m[2]; f11 = m[3];
                }
                if (g_mutant == MUT_ROPE_SIGN) f01 = -f01;
                if (g_mutant == MUT_TABLE_T) { const double t = f01; f01 = f10; f10 = t; }
                const double x0 = n[a], x1 = n[b];
                n[a] = f00 * x0 + f01 * x1;
                n[b] = f10 * x0 + f11 * x1;
            }
        }
        for (int d = 0; d < LRO_D; ++d) yr[d] = (float)n[d];
    }
}

void lro_rms_rope(const uint16_t* x, int64_t rows, int heads, int64_t x_rs, const float* w, const uint16_t* w_bf16,
                  int table_kind, const void* ta, const void* tb, int64_t tab_stride, int pairing, int rot,
                  float eps, float* y) {
    lro_rms_rope_ex(x, rows, heads, x_rs, w, w_bf16, table_kind, ta, tb, tab_stride, pairing, rot, eps, 0, y);
}

static inline int kv_head(int h, int H, int HK) {
    if (g_mutant == MUT_GQA_MOD) return h % HK;
    return h / (H / HK);
}

static inline int visible(int64_t j, int64_t i, int p0, int64_t nkeys, int causal) {
    if (j >= nkeys) return 0;
    if (!causal) return 1;
    if (g_mutant == MUT_CAUSAL_OFF1) return j < (int64_t)p0 + i;
    return j <= (int64_t)p0 + i;
}

/* ---------------------------------------------------------------- attention, fp64 brute force (the pin)
 * q [W][H][128] fp32 dense, k, v [nkeys][HK][128] fp32 dense; out [W][H][128] fp32 dense.
 * A row with no visible key gives 0 (the reference's kernel would divide 0 by 0; callers never ask for it). */
void lro_attention_f64(const float* q, const float* k, const float* v, float* out, int p0, int W, int H, int HK,
                       int nkeys, int causal, float scale) {
    const double sc = g_mutant == MUT_NO_SCALE ? 1.0 : (double)scale;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t ih = 0; ih < (int64_t)W * H; ++ih) {
        const int64_t i = ih / H;
        const int h = (int)(ih % H), hk = kv_head(h, H, HK);
        const float* qi = q + ih * LRO_D;
        double* s = (double*)malloc(sizeof(double) * (size_t)(nkeys > 0 ? nkeys : 1));
        double m = -INFINITY;
        for (int64_t j = 0; j < nkeys; ++j) {
            if (!visible(j, i, p0, nkeys, causal)) { s[j] = -INFINITY; continue; }
            const float* kj = k + (j * HK + hk) * LRO_D;
            double dot = 0.0;
            for (int d = 0; d < LRO_D; ++d) dot += (double)qi[d] * (double)kj[d];
            s[j] = dot * sc;
            if (s[j] > m) m = s[j];
        }
        double o[LRO_D] = {0}, l = 0.0;
        if (m != -INFINITY) {
            for (int64_t j = 0; j < nkeys; ++j) {
                if (s[j] == -INFINITY) continue;
                const double p = exp(s[j] - m);
                l += p;
                const float* vj = v + (j * HK + hk) * LRO_D;
                for (int d = 0; d < LRO_D; ++d) o[d] += p * (double)vj[d];
            }
        }
        float* oi = out + ih * LRO_D;
        for (int d = 0; d < LRO_D; ++d) oi[d] = l > 0.0 ? (float)(o[d] / l) : 0.0f;
        free(s);
    }
}

/* ---------------------------------------------------------------- attention, fp32 flash-style (the CPU baseline)
 * Same contract as lro_attention_f64 but with explicit row strides for q/out (rows of H heads) and k/v (rows of HK
 * heads), and `rows` / `nrows` selecting a subset of query rows: query row rows[r] (or r when rows is NULL) for
 * r < nrows; out row r. Blocks of 32 queries x 64 keys, online softmax in fp32. */
#define BQ 32
#define BK 64
void lro_attention_f32(const float* q, const float* k, const float* v, float* out, int p0, int W, int H, int HK,
                       int nkeys, int causal, float scale, const int64_t* rows, int64_t nrows) {
    const float sc = g_mutant == MUT_NO_SCALE ? 1.0f : scale;
    if (!rows) nrows = W;
    const int64_t qblocks = (nrows + BQ - 1) / BQ;
#pragma omp parallel for schedule(dynamic, 1) collapse(2)
    for (int h = 0; h < H; ++h) {
        for (int64_t qb = 0; qb < qblocks; ++qb) {
            const int hk = kv_head(h, H, HK);
            const int64_t r0 = qb * BQ, nq = (nrows - r0) < BQ ? (nrows - r0) : BQ;
            float qt[BQ][LRO_D], o[BQ][LRO_D], m[BQ], l[BQ], s[BQ][BK];
            int64_t qi[BQ];
            int64_t jmax = nkeys;
            for (int r = 0; r < BQ; ++r) {
                qi[r] = r < nq ? (rows ? rows[r0 + r] : r0 + r) : -1;
                m[r] = -INFINITY;
                l[r] = 0.0f;
                for (int d = 0; d < LRO_D; ++d) {
                    qt[r][d] = r < nq ? q[(qi[r] * H + h) * LRO_D + d] : 0.0f;
                    o[r][d] = 0.0f;
                }
            }
            for (int64_t j0 = 0; j0 < jmax; j0 += BK) {
                const int nk = (jmax - j0) < BK ? (int)(jmax - j0) : BK;
                for (int r = 0; r < nq; ++r) {
                    float tm = -INFINITY;
                    for (int c = 0; c < nk; ++c) {
                        const float* kj = k + ((j0 + c) * HK + hk) * LRO_D;
                        float dot = 0.0f;
#pragma omp simd reduction(+ : dot)
                        for (int d = 0; d < LRO_D; ++d) dot += qt[r][d] * kj[d];
                        s[r][c] = visible(j0 + c, qi[r], p0, nkeys, causal) ? dot * sc : -INFINITY;
                        if (s[r][c] > tm) tm = s[r][c];
                    }
                    const float mn = tm > m[r] ? tm : m[r];
                    if (mn == -INFINITY) continue;
                    const float a = m[r] == -INFINITY ? 0.0f : expf(m[r] - mn);
                    float ls = 0.0f;
                    for (int c = 0; c < nk; ++c) {
                        s[r][c] = s[r][c] == -INFINITY ? 0.0f : expf(s[r][c] - mn);
                        ls += s[r][c];
                    }
                    l[r] = l[r] * a + ls;
                    m[r] = mn;
#pragma omp simd
                    for (int d = 0; d < LRO_D; ++d) o[r][d] *= a;
                    for (int c = 0; c < nk; ++c) {
                        const float p = s[r][c];
                        if (p == 0.0f) continue;
                        const float* vj = v + ((j0 + c) * HK + hk) * LRO_D;
#pragma omp simd
                        for (int d = 0; d < LRO_D; ++d) o[r][d] += p * vj[d];
                    }
                }
            }
            for (int r = 0; r < nq; ++r)
                for (int d = 0; d < LRO_D; ++d)
                    out[((r0 + r) * H + h) * LRO_D + d] = l[r] > 0.0f ? o[r][d] / l[r] : 0.0f;
        }
    }
}

/* ---------------------------------------------------------------- the fused op (Appendix of the build's op definition)
 * q_raw [Sq][H][128] bf16 (row stride q_rs), k_raw [Sk][HK][128] bf16 (row stride k_rs), v [Sk][HK][128] bf16
 * (row stride v_rs). Query row i uses q-table row i; key row j >= n_pre uses k-table row j - n_pre; key rows
 * j < n_pre are taken as already normalised and rotated. Output fp32 [Sq][H][128] dense.
 * precise != 0: fp64 brute-force attention; else the fp32 flash-style path. */
/* round_prepared != 0: the normalised, rotated q and k rounded to bf16 before the attention, as the reference's chain
 * stores them (rope_q / rope_k write bf16 rows that Ops.attention reads, src/engines/qwen_image/dit.zig:252-263). */
void lro_joint_attention_ex(const uint16_t* q_raw, const uint16_t* k_raw, const uint16_t* v, int64_t q_rs,
                            int64_t k_rs, int64_t v_rs, const float* wq, const float* wk, int table_kind,
                            const void* qa, const void* qb, const void* ka, const void* kb, int64_t tab_stride,
                            int pairing, int rot, float eps, int Sq, int Sk, int H, int HK, int p0, int causal,
                            float scale, int n_pre, int precise, int round_prepared, float* out) {
    if (g_mutant == MUT_NO_ROUND_PREP) round_prepared = 0;
    float* qh = (float*)malloc(sizeof(float) * (size_t)Sq * H * LRO_D);
    float* kh = (float*)malloc(sizeof(float) * (size_t)Sk * HK * LRO_D);
    float* vf = (float*)malloc(sizeof(float) * (size_t)Sk * HK * LRO_D);
    lro_rms_rope(q_raw, Sq, H, q_rs, wq, NULL, table_kind, qa, qb, tab_stride, pairing, rot, eps, qh);
    if (n_pre > 0) {
#pragma omp parallel for schedule(static)
        for (int64_t j = 0; j < n_pre; ++j)
            for (int64_t e = 0; e < (int64_t)HK * LRO_D; ++e) kh[j * HK * LRO_D + e] = lro_bf16_to_f32(k_raw[j * k_rs + e]);
    }
    if (Sk > n_pre)
        lro_rms_rope(k_raw + (int64_t)n_pre * k_rs, Sk - n_pre, HK, k_rs, wk, NULL, table_kind, ka, kb, tab_stride,
                     pairing, rot, eps, kh + (int64_t)n_pre * HK * LRO_D);
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < Sk; ++j)
        for (int64_t e = 0; e < (int64_t)HK * LRO_D; ++e) vf[j * HK * LRO_D + e] = lro_bf16_to_f32(v[j * v_rs + e]);
    if (round_prepared) {
        for (int64_t e = 0; e < (int64_t)Sq * H * LRO_D; ++e) qh[e] = lro_bf16_to_f32(lro_f32_to_bf16(qh[e]));
        for (int64_t e = (int64_t)n_pre * HK * LRO_D; e < (int64_t)Sk * HK * LRO_D; ++e)
            kh[e] = lro_bf16_to_f32(lro_f32_to_bf16(kh[e]));
    }
    if (precise)
        lro_attention_f64(qh, kh, vf, out, p0, Sq, H, HK, Sk, causal, scale);
    else
        lro_attention_f32(qh, kh, vf, out, p0, Sq, H, HK, Sk, causal, scale, NULL, 0);
    free(qh);
    free(kh);
    free(vf);
}

void lro_joint_attention(const uint16_t* q_raw, const uint16_t* k_raw, const uint16_t* v, int64_t q_rs, int64_t k_rs,
                         int64_t v_rs, const float* wq, const float* wk, int table_kind, const void* qa, const void* qb,
                         const void* ka, const void* kb, int64_t tab_stride, int pairing, int rot, float eps, int Sq,
                         int Sk, int H, int HK, int p0, int causal, float scale, int n_pre, int precise, float* out) {
    lro_joint_attention_ex(q_raw, k_raw, v, q_rs, k_rs, v_rs, wq, wk, table_kind, qa, qb, ka, kb, tab_stride, pairing,
                           rot, eps, Sq, Sk, H, HK, p0, causal, scale, n_pre, precise, 0, out);
}
