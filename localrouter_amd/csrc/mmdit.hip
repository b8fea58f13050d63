// The MMDiT double-stream block forward (include/lr_mmdit.h): hipBLASLt GEMMs for the projections and the MLP, the
// joint attention of this library (norm + RoPE fused), and HBM-bound HIP kernels for the rest: the time sinusoid,
// SiLU, LayerNorm + adaLN modulation, GELU-tanh and the gated residual. Every kernel reads and writes bf16 rows with
// 16-byte accesses and computes in fp32.
//
// The reference has no double-stream block; its elementwise arithmetic is followed where it has one: the time
// sinusoid (kernels/cuda/qwen_image/ops.cu:84-99), GELU-tanh in torch's operation order (ops.cu:48-57), the gated
// residual x = fma(a, g, x) (ops.cu:25-31) and SiLU x / (1 + exp(-x)) (ops.cu:34-39).
#include <hipblaslt/hipblaslt.h>

#include <cmath>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "../../include/lr_mmdit.h"
#include "lr_common.h"

namespace lr {
namespace {

constexpr int EW_THREADS = 256;
constexpr size_t GEMM_WS = LR_MMDIT_GEMM_WORKSPACE;   // hipBLASLt workspace, at the start of the block's scratch
constexpr float LN_EPS = 1e-6f;

__device__ __forceinline__ float bf(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ uint16_t tobf(float f) { return __builtin_bit_cast(uint16_t, (bf16)f); }

// emb[256] from t (ops.cu:84-99): t scaled by 1000 and rounded to bf16, divided by 1000 (reciprocal multiply) and
// rounded again, times 1000; freq_i = exp(-ln(10000) i / 128); cos for j < 128, sin for j >= 128.
__device__ __forceinline__ float time_scaled(const float* t) {
    float tr = bf(tobf(t[0] * 1000.0f));
    tr = bf(tobf(tr * (1.0f / 1000.0f)));
    return tr * 1000.0f;
}
__device__ __forceinline__ uint16_t sinusoid_at(float tr, int j) {
    const int i = j & 127;
    const float c = -9.210340371976184f;   // -ln(10000)
    const float freq = expf((c * (float)i) * (1.0f / 128.0f));
    const float arg = tr * freq;
    return tobf(j < 128 ? cosf(arg) : sinf(arg));
}
__global__ void time_sinusoid_kernel(const float* t, uint16_t* emb) {
    emb[threadIdx.x] = sinusoid_at(time_scaled(t), threadIdx.x);
}

// y = x / (1 + exp(-x)), n elements (small vectors)
__global__ void silu_kernel(const uint16_t* x, uint16_t* y, int n) {
    const int i = blockIdx.x * EW_THREADS + threadIdx.x;
    if (i >= n) return;
    const float v = bf(x[i]);
    y[i] = tobf(v / (1.0f + expf(-v)));
}

struct Chunk8 {
    float v[8];
};
__device__ __forceinline__ Chunk8 load8(const uint16_t* p) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(p);
    Chunk8 c;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        c.v[2 * k] = lo_bf16(w[k]);
        c.v[2 * k + 1] = hi_bf16(w[k]);
    }
    return c;
}
__device__ __forceinline__ void store8(uint16_t* p, const Chunk8& c) {
    u32x4 w;
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = pack_bf16x2(c.v[2 * k], c.v[2 * k + 1]);
    *reinterpret_cast<u32x4*>(p) = w;
}

// Row sums over a workgroup of LN_THREADS: wave butterflies, then the waves' partials through LDS.
constexpr int LN_THREADS = 256;
constexpr int LN_MAX_CHUNKS = 4;   // D <= 8 * LN_THREADS * LN_MAX_CHUNKS = 8192
__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();   // red is reused by consecutive sums
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < LN_THREADS / 64; ++w) s += red[w];
    return s;
}

// out row r (txt rows 0..n_txt-1, then img rows) = LayerNorm(x_r) * (1 + scale) + shift with the row's stream's
// modulation chunk (shift = mod[which * 3 D .. + D), scale = the next D), two-pass mean and variance in fp32.
// RES: first the gated residual of the half before, x_r += g * a_r (gated_residual_kernel's arithmetic, g the gate
// chunk of `res_which`), x_r stored and normalised as the bf16 values stored. out may be a (each workgroup reads its
// whole row of a before the first barrier and writes out after the second).
template <bool RES>
__global__ __launch_bounds__(LN_THREADS) void ln_modulate_kernel(uint16_t* txt, uint16_t* img, int n_txt, int D,
                                                                 const uint16_t* mod_txt, const uint16_t* mod_img,
                                                                 int which, uint16_t* out, const uint16_t* a,
                                                                 int res_which) {
    __shared__ float red[LN_THREADS / 64];
    const int r = blockIdx.x;
    const bool is_txt = r < n_txt;
    uint16_t* x = is_txt ? txt + (int64_t)r * D : img + (int64_t)(r - n_txt) * D;
    const uint16_t* mod = (is_txt ? mod_txt : mod_img) + (int64_t)which * 3 * D;
    const int chunks = D / 8;
    Chunk8 c[LN_MAX_CHUNKS];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < LN_MAX_CHUNKS; ++k) {
        const int ch = threadIdx.x + k * LN_THREADS;
        if (ch < chunks) {
            c[k] = load8(x + 8 * ch);
            if constexpr (RES) {
                const uint16_t* g = (is_txt ? mod_txt : mod_img) + (int64_t)res_which * 3 * D + 2 * D;
                const Chunk8 av = load8(a + (int64_t)r * D + 8 * ch), gv = load8(g + 8 * ch);
#pragma unroll
                for (int e = 0; e < 8; ++e) c[k].v[e] = bf(tobf(fmaf(av.v[e], gv.v[e], c[k].v[e])));   // as stored
                store8(x + 8 * ch, c[k]);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) s += c[k].v[e];
        }
    }
    const float mean = block_sum(s, red) / (float)D;
    float q = 0.0f;
#pragma unroll
    for (int k = 0; k < LN_MAX_CHUNKS; ++k) {
        const int ch = threadIdx.x + k * LN_THREADS;
        if (ch < chunks) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float d = c[k].v[e] - mean;
                q += d * d;
            }
        }
    }
    const float rstd = rsqrtf(block_sum(q, red) / (float)D + LN_EPS);
    uint16_t* y = out + (int64_t)r * D;
#pragma unroll
    for (int k = 0; k < LN_MAX_CHUNKS; ++k) {
        const int ch = threadIdx.x + k * LN_THREADS;
        if (ch < chunks) {
            const Chunk8 sh = load8(mod + 8 * ch), sc = load8(mod + D + 8 * ch);
            Chunk8 o;
#pragma unroll
            for (int e = 0; e < 8; ++e) o.v[e] = (c[k].v[e] - mean) * rstd * (1.0f + sc.v[e]) + sh.v[e];
            store8(y + 8 * ch, o);
        }
    }
}

// x = 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) in place, torch's order (ops.cu:48-57); n8 chunks of 8.
__global__ void gelu_tanh_kernel(uint16_t* x, int64_t n8) {
    const int64_t i = (int64_t)blockIdx.x * EW_THREADS + threadIdx.x;
    if (i >= n8) return;
    const float kBeta = (float)(1.4142135623730951 * 1.1283791670955126 * 0.5);
    const float kKappa = 0.044715f;
    Chunk8 c = load8(x + 8 * i);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float v = c.v[e];
        const float cube = v * v * v;
        const float inner = kBeta * fmaf(kKappa, cube, v);
        c.v[e] = (0.5f * v) * (1.0f + tanhf(inner));
    }
    store8(x + 8 * i, c);
}

// x_r += g * a_r (fma(a, g, x), ops.cu:25-31) for the joint rows, g the row's stream's gate chunk
// (mod[which * 3 D + 2 D .. + D)); one 8-element chunk per thread.
__global__ void gated_residual_kernel(uint16_t* txt, uint16_t* img, int n_txt, int n_rows, int D, const uint16_t* a,
                                      const uint16_t* mod_txt, const uint16_t* mod_img, int which) {
    const int chunks = D / 8;
    const int64_t i = (int64_t)blockIdx.x * EW_THREADS + threadIdx.x;
    if (i >= (int64_t)n_rows * chunks) return;
    const int r = (int)(i / chunks), ch = (int)(i - (int64_t)r * chunks);
    const bool is_txt = r < n_txt;
    uint16_t* x = is_txt ? txt + (int64_t)r * D : img + (int64_t)(r - n_txt) * D;
    const uint16_t* g = (is_txt ? mod_txt : mod_img) + (int64_t)which * 3 * D + 2 * D;
    Chunk8 xv = load8(x + 8 * ch);
    const Chunk8 av = load8(a + (int64_t)r * D + 8 * ch), gv = load8(g + 8 * ch);
#pragma unroll
    for (int e = 0; e < 8; ++e) xv.v[e] = fmaf(av.v[e], gv.v[e], xv.v[e]);
    store8(x + 8 * ch, xv);
}

// The gated residual of rows whose down-projection ran as KSPLIT slices: a = bf16(sum of the slices' fp32 partials, in
// slice order), as the unsliced GEMM's bf16 output; then x = fma(a, g, x) as gated_residual_kernel. part is
// [KSPLIT][rows][D] fp32, g the gate chunk (mod[which * 3 D + 2 D .. + D)); one 8-element chunk per thread.
__global__ void ksum_residual_kernel(uint16_t* x, const float* part, int rows, int D, const uint16_t* mod, int which,
                                     int nslices) {
    const int chunks = D / 8;
    const int64_t i = (int64_t)blockIdx.x * EW_THREADS + threadIdx.x;
    if (i >= (int64_t)rows * chunks) return;
    const int64_t slice = (int64_t)rows * D, off = 8 * i;   // element offset of this chunk in one slice
    f32x4 s0 = *reinterpret_cast<const f32x4*>(part + off), s1 = *reinterpret_cast<const f32x4*>(part + off + 4);
    for (int j = 1; j < nslices; ++j) {
        s0 += *reinterpret_cast<const f32x4*>(part + j * slice + off);
        s1 += *reinterpret_cast<const f32x4*>(part + j * slice + off + 4);
    }
    const int64_t r = i / chunks, ch = i - r * chunks;
    uint16_t* xr = x + r * D + 8 * ch;
    const Chunk8 gv = load8(mod + (int64_t)which * 3 * D + 2 * D + 8 * ch);
    Chunk8 xv = load8(xr);
#pragma unroll
    for (int e = 0; e < 8; ++e) xv.v[e] = fmaf(bf(tobf(e < 4 ? s0[e] : s1[e - 4])), gv.v[e], xv.v[e]);
    store8(xr, xv);
}

// y[n] = sum_k x[k] w[n, k] for one input row (the time and modulation vectors): HBM-bound on w, one wave per
// output, 16-byte loads along the weight row, a butterfly sum. K a multiple of 8. SILU: y = SiLU of the bf16 result,
// the arithmetic of silu_kernel (the time MLP's two activations without launches of their own). SIN: x is the time
// sinusoid of *t (K = 256), each element computed where it is used, as time_sinusoid_kernel computes it.
constexpr int GEMV_WAVES = 4;
template <bool SILU, bool SIN = false>
__global__ __launch_bounds__(64 * GEMV_WAVES) void gemv_kernel(const uint16_t* x, const uint16_t* w, uint16_t* y, int N,
                                                               int K, const float* t = nullptr) {
    const int n = blockIdx.x * GEMV_WAVES + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (n >= N) return;
    const uint16_t* row = w + (int64_t)n * K;
    float tr = 0.0f;
    if constexpr (SIN) tr = time_scaled(t);
    float acc = 0.0f;
    for (int c = lane; c < K / 8; c += 64) {
        const Chunk8 a = load8(row + 8 * c);
        Chunk8 b;
        if constexpr (SIN) {
#pragma unroll
            for (int e = 0; e < 8; ++e) b.v[e] = bf(sinusoid_at(tr, 8 * c + e));
        } else {
            b = load8(x + 8 * c);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = fmaf(a.v[e], b.v[e], acc);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (lane == 0) {
        if constexpr (SILU) {
            const float v = bf(tobf(acc));
            y[n] = tobf(v / (1.0f + expf(-v)));
        } else {
            y[n] = tobf(acc);
        }
    }
}

// ---- hipBLASLt GEMMs: row-major Y[M, N] (row stride ldy) = X[M, K] (row stride ldx) W[N, K]^T, bf16 in and out,
// fp32 compute. Column-major, that is C (N x M, ldc = ldy) = op(A) op(B) with A = W viewed K x N (lda = K,
// transposed) and B = X viewed K x M (ldb = ldx).
struct GemmPlan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    size_t ws = 0;
};
// M, N, K, ldx, ldy, epilogue (EPI_NONE, or EPI_GELU: y = GELU(x w^T) applied to the fp32 result before the bf16
// store, hipBLASLt's GELU epilogue, which takes the place of gelu_tanh_kernel for the MLP up-projection)
using GemmKey = std::tuple<int64_t, int64_t, int64_t, int64_t, int64_t, int>;
constexpr int EPI_NONE = 0, EPI_GELU = 1, EPI_KSPLIT = 2;
// EPI_KSPLIT: the down-projection of a stream of at most KSPLIT_ROWS rows as one strided-batched GEMM over KSPLIT
// slices of K with fp32 partials (row-major [slice][M][N]), summed by ksum_residual_kernel: a 512-row down-projection
// alone gives hipBLASLt too few output tiles for the 256 CUs.
constexpr int KSPLIT = 4;
constexpr int64_t KSPLIT_ROWS = 1024;
bool ksplit_rows(int64_t M, int64_t F) { return M > 1 && M <= KSPLIT_ROWS && F % (8 * KSPLIT) == 0; }

// A context's plans are built by lr_mmdit_plan / lr_mmdit_tune (and by lr_mmdit_linear_bf16 for a new shape) under
// `mu`; the block call only looks them up. A plan is never removed before the context is destroyed, so a pointer to
// it stays valid.
struct Ctx {
    hipblasLtHandle_t lt = nullptr;
    std::map<GemmKey, GemmPlan> plans;
    std::mutex mu;
};

int blas_err(hipblasStatus_t s) { return s == HIPBLAS_STATUS_SUCCESS ? 0 : 1000 + (int)s; }

void destroy_plan(GemmPlan& p) {
    if (p.la) hipblasLtMatrixLayoutDestroy(p.la);
    if (p.lb) hipblasLtMatrixLayoutDestroy(p.lb);
    if (p.lc) hipblasLtMatrixLayoutDestroy(p.lc);
    if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
    p = GemmPlan{};
}

// The plan of one GEMM shape, if built (caller holds c.mu or only reads a map no one is changing).
GemmPlan* find_plan(Ctx& c, int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldy, int epi = EPI_NONE) {
    auto it = c.plans.find(GemmKey{M, N, K, ldx, ldy, epi});
    return it == c.plans.end() ? nullptr : &it->second;
}

// Build (heuristic-first) and keep the plan of one GEMM shape; every handle created on a failed path is destroyed.
// A GELU plan for which hipBLASLt has no algorithm fails with 1000 + HIPBLAS_STATUS_NOT_SUPPORTED.
int plan_gemm(Ctx& c, int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldy, int epi, GemmPlan** out) {
    std::lock_guard<std::mutex> lock(c.mu);
    if (GemmPlan* found = find_plan(c, M, N, K, ldx, ldy, epi)) {
        *out = found;
        return 0;
    }
    GemmPlan p;
    hipblasLtMatmulPreference_t pref = nullptr;
    auto fail = [&](int rc) {
        if (pref) hipblasLtMatmulPreferenceDestroy(pref);
        destroy_plan(p);
        return rc;
    };
    int rc;
    if ((rc = blas_err(hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F)))) return fail(rc);
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    if ((rc = blas_err(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta))))
        return fail(rc);
    if ((rc = blas_err(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb))))
        return fail(rc);
    if (epi == EPI_GELU) {
        const hipblasLtEpilogue_t e = HIPBLASLT_EPILOGUE_GELU;
        if ((rc = blas_err(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &e, sizeof e))))
            return fail(rc);
    }
    const int64_t Ks = epi == EPI_KSPLIT ? K / KSPLIT : K;
    if ((rc = blas_err(hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16BF, Ks, N, K)))) return fail(rc);
    if ((rc = blas_err(hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_16BF, Ks, M, ldx)))) return fail(rc);
    if ((rc = blas_err(hipblasLtMatrixLayoutCreate(&p.lc, epi == EPI_KSPLIT ? HIP_R_32F : HIP_R_16BF, N, M, ldy))))
        return fail(rc);
    if (epi == EPI_KSPLIT) {   // slice i: K columns [i Ks, (i + 1) Ks) of W and X, partial i at i M N floats
        const int32_t bc = KSPLIT;
        const int64_t sa = Ks, sb = Ks, sc = N * M;
        for (hipblasLtMatrixLayout_t l : {p.la, p.lb, p.lc})
            if ((rc = blas_err(hipblasLtMatrixLayoutSetAttribute(l, HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &bc, sizeof bc))))
                return fail(rc);
        if ((rc = blas_err(hipblasLtMatrixLayoutSetAttribute(p.la, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &sa,
                                                             sizeof sa))) ||
            (rc = blas_err(hipblasLtMatrixLayoutSetAttribute(p.lb, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &sb,
                                                             sizeof sb))) ||
            (rc = blas_err(hipblasLtMatrixLayoutSetAttribute(p.lc, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &sc,
                                                             sizeof sc))))
            return fail(rc);
    }
    if ((rc = blas_err(hipblasLtMatmulPreferenceCreate(&pref)))) return fail(rc);
    const uint64_t ws = GEMM_WS;
    if ((rc = blas_err(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                                             sizeof ws))))
        return fail(rc);
    hipblasLtMatmulHeuristicResult_t res[1];
    int found = 0;
    if ((rc = blas_err(hipblasLtMatmulAlgoGetHeuristic(c.lt, p.desc, p.la, p.lb, p.lc, p.lc, pref, 1, res, &found))))
        return fail(rc);
    if (found < 1) return fail(1000 + (int)HIPBLAS_STATUS_NOT_SUPPORTED);
    hipblasLtMatmulPreferenceDestroy(pref);
    p.algo = res[0].algo;
    p.ws = res[0].workspaceSize;
    auto ins = c.plans.emplace(GemmKey{M, N, K, ldx, ldy, epi}, p);
    *out = &ins.first->second;
    return 0;
}

// Time up to `cands` heuristic candidates of one GEMM on the given buffers and keep the fastest as its plan
// (replacing a heuristic-first plan). Synchronises on its own events.
int tune_gemm(Ctx& c, const void* X, int64_t ldx, const void* W, void* Y, int64_t ldy, int64_t M, int64_t N,
              int64_t K, int epi, void* ws, hipStream_t s, int cands) {
    GemmPlan* p;
    int rc = plan_gemm(c, M, N, K, ldx, ldy, epi, &p);
    if (rc) return rc;
    hipblasLtMatmulPreference_t pref;
    if ((rc = blas_err(hipblasLtMatmulPreferenceCreate(&pref)))) return rc;
    const uint64_t wsb = GEMM_WS;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb, sizeof wsb);
    hipblasLtMatmulHeuristicResult_t res[16];
    int found = 0;
    cands = cands > 16 ? 16 : cands;
    rc = blas_err(hipblasLtMatmulAlgoGetHeuristic(c.lt, p->desc, p->la, p->lb, p->lc, p->lc, pref, cands, res, &found));
    hipblasLtMatmulPreferenceDestroy(pref);
    if (rc) return rc;
    hipEvent_t e0, e1;
    if ((rc = (int)hipEventCreate(&e0))) return rc;
    if ((rc = (int)hipEventCreate(&e1))) {
        (void)hipEventDestroy(e0);
        return rc;
    }
    const float alpha = 1.0f, beta = 0.0f;
    float best = 1e30f;
    for (int i = 0; i < found && rc == 0; ++i) {
        if (res[i].workspaceSize > GEMM_WS) continue;
        auto run = [&]() {
            return hipblasLtMatmul(c.lt, p->desc, &alpha, W, p->la, X, p->lb, &beta, Y, p->lc, Y, p->lc, &res[i].algo,
                                   ws, res[i].workspaceSize, s);
        };
        if (run() != HIPBLAS_STATUS_SUCCESS) continue;   // a candidate that does not run is skipped
        (void)hipEventRecord(e0, s);
        for (int r = 0; r < 5; ++r) run();
        (void)hipEventRecord(e1, s);
        if ((rc = (int)hipEventSynchronize(e1))) break;
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, e0, e1);
        if (ms < best) {
            best = ms;
            std::lock_guard<std::mutex> lock(c.mu);
            p->algo = res[i].algo;
            p->ws = res[i].workspaceSize;
        }
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return rc;
}

bool is_vector(int64_t M, int64_t K, const void* X, const void* W) {
    return M == 1 && K % 8 == 0 && ((uintptr_t)X & 15) == 0 && ((uintptr_t)W & 15) == 0;
}

// One GEMM on the stream. plan_new: build the shape's plan if missing (lr_mmdit_linear_bf16); otherwise the plan must
// exist (the block call, which checked every plan before its first launch).
int gemm(Ctx& c, const void* X, int64_t ldx, const void* W, void* Y, int64_t ldy, int64_t M, int64_t N, int64_t K,
         void* ws, hipStream_t s, bool plan_new = false, int epi = EPI_NONE) {
    if (is_vector(M, K, X, W)) {   // a vector: HBM-bound
        hipLaunchKernelGGL(gemv_kernel<false>, dim3((unsigned)((N + GEMV_WAVES - 1) / GEMV_WAVES)), dim3(64 * GEMV_WAVES), 0,
                           s, static_cast<const uint16_t*>(X), static_cast<const uint16_t*>(W),
                           static_cast<uint16_t*>(Y), (int)N, (int)K);
        return (int)hipGetLastError();
    }
    GemmPlan* p = nullptr;
    int rc = 0;
    if (plan_new) {
        rc = plan_gemm(c, M, N, K, ldx, ldy, epi, &p);
    } else {
        std::lock_guard<std::mutex> lock(c.mu);
        p = find_plan(c, M, N, K, ldx, ldy, epi);
        if (!p) rc = (int)hipErrorNotReady;
    }
    if (rc) return rc;
    const float alpha = 1.0f, beta = 0.0f;
    return blas_err(hipblasLtMatmul(c.lt, p->desc, &alpha, W, p->la, X, p->lb, &beta, Y, p->lc, Y, p->lc, &p->algo, ws,
                                    p->ws, s));
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// The row GEMMs of one block call (M > 1: the vectors go to gemv_kernel): QKV, out, MLP up and down, per stream of rows,
// as {M, N, K, ldx, ldy, epilogue}. The up-projection is listed with its GELU epilogue; a context where hipBLASLt has no
// algorithm for that holds the plain plan instead and the block applies gelu_tanh_kernel (up_epi).
std::vector<GemmKey> block_gemms(int64_t n_txt, int64_t n_img, int64_t D, int64_t F) {
    std::vector<GemmKey> g;
    for (const int64_t M : {n_txt, n_img}) {
        if (M <= 1) continue;
        g.push_back(GemmKey{M, 3 * D, D, D, 3 * D, EPI_NONE});
        g.push_back(GemmKey{M, D, D, D, D, EPI_NONE});
        g.push_back(GemmKey{M, F, D, D, F, EPI_GELU});
        g.push_back(ksplit_rows(M, F) ? GemmKey{M, D, F, F, D, EPI_KSPLIT} : GemmKey{M, D, F, F, D, EPI_NONE});
    }
    return g;
}

// The epilogue the context's plan of an up-projection shape has: EPI_GELU when hipBLASLt had an algorithm for it,
// else EPI_NONE (-1: neither is planned). Caller holds c.mu.
int up_epi(Ctx& c, int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldy) {
    if (find_plan(c, M, N, K, ldx, ldy, EPI_GELU)) return EPI_GELU;
    return find_plan(c, M, N, K, ldx, ldy, EPI_NONE) ? EPI_NONE : -1;
}
// Likewise for a down-projection: EPI_KSPLIT when its stream qualifies and the sliced plan exists, else EPI_NONE.
int down_epi(Ctx& c, int64_t M, int64_t D, int64_t F) {
    if (ksplit_rows(M, F) && find_plan(c, M, D, F, F, D, EPI_KSPLIT)) return EPI_KSPLIT;
    return find_plan(c, M, D, F, F, D, EPI_NONE) ? EPI_NONE : -1;
}

// Plan one block GEMM; the up-projection falls back to the plain plan (and gelu_tanh_kernel) when hipBLASLt has no
// algorithm with the GELU epilogue for it, a sliced down-projection to the plain plan when it has none for the slices.
int plan_block_gemm(Ctx& c, const GemmKey& k) {
    GemmPlan* p;
    int rc = plan_gemm(c, std::get<0>(k), std::get<1>(k), std::get<2>(k), std::get<3>(k), std::get<4>(k),
                       std::get<5>(k), &p);
    if (rc && (std::get<5>(k) == EPI_GELU || std::get<5>(k) == EPI_KSPLIT))
        rc = plan_gemm(c, std::get<0>(k), std::get<1>(k), std::get<2>(k), std::get<3>(k), std::get<4>(k), EPI_NONE, &p);
    return rc;
}

// scratch layout of one block call
struct Scratch {
    size_t emb, h1, temb, ts, mod_txt, mod_img, hn, qkv, attn, big, gws, attn_ws, kpart_txt, kpart_img, total;
};
Scratch layout(int64_t n_txt, int64_t n_img, int64_t D, int64_t F) {
    const int64_t S = n_txt + n_img;
    Scratch s;
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o += align256(bytes);
        return at;
    };
    s.gws = take(GEMM_WS);
    s.emb = take(256 * 2);
    s.h1 = take(D * 2);
    s.temb = take(D * 2);
    s.ts = take(D * 2);
    s.mod_txt = take(6 * D * 2);
    s.mod_img = take(6 * D * 2);
    s.hn = take(S * D * 2);          // LayerNorm + modulation, then the out projection, then the MLP output
    s.qkv = take(S * 3 * D * 2);
    s.attn = take(S * D * 2);        // attention output
    s.big = take(S * F * 2);         // MLP hidden
    s.attn_ws = take(lr_joint_attention_workspace_bytes((int)S, (int)(D / 128)));
    // the sliced down-projections' fp32 partials (streams that qualify)
    s.kpart_txt = take(ksplit_rows(n_txt, F) ? (size_t)KSPLIT * n_txt * D * 4 : 0);
    s.kpart_img = take(ksplit_rows(n_img, F) ? (size_t)KSPLIT * n_img * D * 4 : 0);
    s.total = o;
    return s;
}

}  // namespace
}  // namespace lr

using namespace lr;

extern "C" {

int lr_mmdit_create(void** ctx) {
    if (!ctx) return hipErrorInvalidValue;
    Ctx* c = new Ctx;
    const int rc = blas_err(hipblasLtCreate(&c->lt));
    if (rc) {
        lr_mmdit_destroy(c);
        return rc;
    }
    *ctx = c;
    return 0;
}

int lr_mmdit_destroy(void* ctx) {
    if (!ctx) return hipErrorInvalidValue;
    Ctx* c = static_cast<Ctx*>(ctx);
    for (auto& kv : c->plans) {
        hipblasLtMatrixLayoutDestroy(kv.second.la);
        hipblasLtMatrixLayoutDestroy(kv.second.lb);
        hipblasLtMatrixLayoutDestroy(kv.second.lc);
        hipblasLtMatmulDescDestroy(kv.second.desc);
    }
    const int rc = c->lt ? blas_err(hipblasLtDestroy(c->lt)) : 0;
    delete c;
    return rc;
}

size_t lr_mmdit_workspace_bytes(int n_txt, int n_img, int hidden, int mlp) {
    if (n_txt < 0 || n_img < 0 || n_txt + n_img <= 0 || hidden <= 0 || hidden % 128 || mlp <= 0 || mlp % 8 ||
        hidden > 8 * LN_THREADS * LN_MAX_CHUNKS)
        return 0;
    return layout(n_txt, n_img, hidden, mlp).total;
}

int lr_mmdit_plan(void* ctx, int n_txt, int n_img, int hidden, int mlp) {
    if (!ctx || lr_mmdit_workspace_bytes(n_txt, n_img, hidden, mlp) == 0) return hipErrorInvalidValue;
    Ctx& c = *static_cast<Ctx*>(ctx);
    for (const GemmKey& k : block_gemms(n_txt, n_img, hidden, mlp)) {
        const int rc = plan_block_gemm(c, k);
        if (rc) return rc;
    }
    return 0;
}

int lr_mmdit_tune(void* ctx, const lr_mmdit_weights* w, int n_txt, int n_img, int hidden, int mlp, int candidates,
                  void* workspace, size_t workspace_bytes, lr_stream_t stream) {
    const size_t need = lr_mmdit_workspace_bytes(n_txt, n_img, hidden, mlp);
    if (!ctx || !w || !workspace || need == 0 || workspace_bytes < need || candidates < 1) return hipErrorInvalidValue;
    if (!w->txt.qkv || !w->txt.out || !w->txt.mlp_up || !w->txt.mlp_down || !w->img.qkv || !w->img.out ||
        !w->img.mlp_up || !w->img.mlp_down)
        return hipErrorInvalidValue;
    Ctx& c = *static_cast<Ctx*>(ctx);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int64_t D = hidden, F = mlp;
    const Scratch L = layout(n_txt, n_img, D, F);
    char* ws = static_cast<char*>(workspace);
    auto at = [&](size_t off) { return reinterpret_cast<uint16_t*>(ws + off); };
    uint16_t *hn = at(L.hn), *qkv = at(L.qkv), *attn = at(L.attn), *big = at(L.big);
    void* gws = ws + L.gws;
    // the block's GEMMs of rows > 1, on its own scratch buffers (contents irrelevant for timing)
    const lr_mmdit_stream_weights* sw[2] = {&w->txt, &w->img};
    const int64_t rows[2] = {n_txt, n_img}, row0[2] = {0, n_txt};
    int rc = 0;
    for (int k = 0; k < 2 && rc == 0; ++k) {
        const int64_t M = rows[k], r0 = row0[k];
        if (M <= 1) continue;
        if (!rc) rc = plan_block_gemm(c, GemmKey{M, F, D, D, F, EPI_GELU});
        int epi = EPI_NONE;
        if (!rc) {
            std::lock_guard<std::mutex> lock(c.mu);
            epi = up_epi(c, M, F, D, D, F);
        }
        if (!rc) rc = tune_gemm(c, hn + r0 * D, D, sw[k]->qkv, qkv + r0 * 3 * D, 3 * D, M, 3 * D, D, EPI_NONE, gws, s,
                                candidates);
        if (!rc) rc = tune_gemm(c, attn + r0 * D, D, sw[k]->out, hn + r0 * D, D, M, D, D, EPI_NONE, gws, s, candidates);
        if (!rc) rc = tune_gemm(c, hn + r0 * D, D, sw[k]->mlp_up, big + r0 * F, F, M, F, D, epi, gws, s, candidates);
        if (!rc)
            rc = plan_block_gemm(c, ksplit_rows(M, F) ? GemmKey{M, D, F, F, D, EPI_KSPLIT} : GemmKey{M, D, F, F, D, EPI_NONE});
        int depi = EPI_NONE;
        if (!rc) {
            std::lock_guard<std::mutex> lock(c.mu);
            depi = down_epi(c, M, D, F);
        }
        void* ydown = depi == EPI_KSPLIT ? (void*)(ws + (k == 0 ? L.kpart_txt : L.kpart_img)) : (void*)(attn + r0 * D);
        if (!rc) rc = tune_gemm(c, big + r0 * F, F, sw[k]->mlp_down, ydown, D, M, D, F, depi, gws, s, candidates);
    }
    return rc;
}

int lr_mmdit_linear_bf16(void* ctx, const void* x, int64_t ldx, const void* w, void* y, int64_t ldy, int M, int N,
                         int K, void* workspace, size_t workspace_bytes, lr_stream_t stream) {
    if (!ctx || !x || !w || !y || !workspace || workspace_bytes < GEMM_WS || M <= 0 || N <= 0 || K <= 0 || ldx < K ||
        ldy < N)
        return hipErrorInvalidValue;
    return gemm(*static_cast<Ctx*>(ctx), x, ldx, w, y, ldy, M, N, K, workspace, reinterpret_cast<hipStream_t>(stream),
                true);
}

int lr_mmdit_block_bf16(void* ctx, const lr_mmdit_weights* w, void* txt, void* img, int n_txt, int n_img, int hidden,
                        int mlp, const float* t, const float* cos, const float* sin, void* workspace,
                        size_t workspace_bytes, lr_stream_t stream) {
    const size_t need = lr_mmdit_workspace_bytes(n_txt, n_img, hidden, mlp);
    if (!ctx || !w || !t || !cos || !sin || !workspace || need == 0 || workspace_bytes < need) return hipErrorInvalidValue;
    if ((n_txt > 0 && !txt) || (n_img > 0 && !img)) return hipErrorInvalidValue;
    const void* ptrs[] = {w->t1, w->t2, w->q_norm, w->k_norm, w->txt.mod, w->txt.qkv, w->txt.out, w->txt.mlp_up,
                          w->txt.mlp_down, w->img.mod, w->img.qkv, w->img.out, w->img.mlp_up, w->img.mlp_down};
    for (const void* p : ptrs)
        if (!p || ((uintptr_t)p & 15) != 0) return hipErrorInvalidValue;
    if ((((uintptr_t)txt | (uintptr_t)img | (uintptr_t)workspace) & 15) != 0) return hipErrorInvalidValue;
    {   // the workspace holds the block's intermediates while txt and img are updated and everything else is read
        const uintptr_t lo = (uintptr_t)workspace, hi = lo + need;
        const size_t D = (size_t)hidden, F = (size_t)mlp, S = (size_t)n_txt + (size_t)n_img;
        const struct { const void* p; size_t bytes; } spans[] = {
            {txt, (size_t)n_txt * D * 2}, {img, (size_t)n_img * D * 2}, {cos, S * 64 * 4}, {sin, S * 64 * 4},
            {t, 4}, {w->t1, D * 256 * 2}, {w->t2, D * D * 2}, {w->q_norm, 128 * 4}, {w->k_norm, 128 * 4},
            {w->txt.mod, 6 * D * D * 2}, {w->txt.qkv, 3 * D * D * 2}, {w->txt.out, D * D * 2},
            {w->txt.mlp_up, F * D * 2}, {w->txt.mlp_down, D * F * 2}, {w->img.mod, 6 * D * D * 2},
            {w->img.qkv, 3 * D * D * 2}, {w->img.out, D * D * 2}, {w->img.mlp_up, F * D * 2},
            {w->img.mlp_down, D * F * 2}};
        for (const auto& sp : spans) {
            const uintptr_t a = (uintptr_t)sp.p;
            if (sp.bytes > 0 && a < hi && lo < a + sp.bytes) return hipErrorInvalidValue;
        }
    }

    Ctx& c = *static_cast<Ctx*>(ctx);
    // every row GEMM's plan exists (lr_mmdit_plan / lr_mmdit_tune), checked before anything is launched; the
    // up-projection of a stream of rows (text 0, image 1) has its GELU fused when its plan carries the epilogue
    bool gelu_fused[2] = {false, false}, ksplit[2] = {false, false};
    {
        std::lock_guard<std::mutex> lock(c.mu);
        const int64_t rows[2] = {n_txt, n_img}, D = hidden, F = mlp;
        for (int k = 0; k < 2; ++k) {
            const int64_t M = rows[k];
            if (M <= 1) continue;   // a vector: gemv_kernel, no plan
            if (!find_plan(c, M, 3 * D, D, D, 3 * D) || !find_plan(c, M, D, D, D, D)) return hipErrorNotReady;
            const int e = up_epi(c, M, F, D, D, F), de = down_epi(c, M, D, F);
            if (e < 0 || de < 0) return hipErrorNotReady;
            gelu_fused[k] = e == EPI_GELU;
            ksplit[k] = de == EPI_KSPLIT;
        }
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int64_t D = hidden, F = mlp, S = (int64_t)n_txt + n_img, H = D / 128;
    const Scratch L = layout(n_txt, n_img, D, F);
    char* ws = static_cast<char*>(workspace);
    auto at = [&](size_t off) { return reinterpret_cast<uint16_t*>(ws + off); };
    uint16_t *emb = at(L.emb), *h1 = at(L.h1), *temb = at(L.temb), *ts = at(L.ts);
    uint16_t *mod_txt = at(L.mod_txt), *mod_img = at(L.mod_img), *hn = at(L.hn), *qkv = at(L.qkv);
    uint16_t *attn = at(L.attn), *big = at(L.big);
    void* gws = ws + L.gws;
    uint16_t* xt = static_cast<uint16_t*>(txt);
    uint16_t* xi = static_cast<uint16_t*>(img);
    int rc;
#define LR_TRY(expr)                     \
    do {                                 \
        if ((rc = (expr)) != 0) return rc; \
    } while (0)
#define LR_LAUNCHED() LR_TRY((int)hipGetLastError())
    // one GEMM per stream of rows, each with its own weights (the text rows first in every joint buffer). Running
    // the text rows' GEMMs on a second stream beside the image rows' was measured slower (1.50 vs 1.34 ms a block).
    auto pair_gemm = [&](const uint16_t* xt_, const uint16_t* xi_, int64_t ldx, const void* wt, const void* wi,
                         uint16_t* yt, uint16_t* yi, int64_t ldy, int64_t N, int64_t K) -> int {
        int r = 0;
        if (n_txt > 0) r = gemm(c, xt_, ldx, wt, yt, ldy, n_txt, N, K, gws, s);
        if (!r && n_img > 0) r = gemm(c, xi_, ldx, wi, yi, ldy, n_img, N, K, gws, s);
        return r;
    };

    // time embedding and modulation (vectors: one row)

    // linear -> SiLU twice: the GEMV applies the SiLU when it serves the vector (aligned, K a multiple of 8)
    auto linear_silu = [&](const uint16_t* x_, const void* w_, uint16_t* pre, uint16_t* y_, int64_t N, int64_t K) -> int {
        if (is_vector(1, K, x_, w_)) {
            hipLaunchKernelGGL(gemv_kernel<true>, dim3((unsigned)((N + GEMV_WAVES - 1) / GEMV_WAVES)),
                               dim3(64 * GEMV_WAVES), 0, s, x_, static_cast<const uint16_t*>(w_), y_, (int)N, (int)K);
            return (int)hipGetLastError();
        }
        int r = gemm(c, x_, K, w_, pre, N, 1, N, K, gws, s);
        if (r) return r;
        hipLaunchKernelGGL(silu_kernel, dim3((unsigned)((N + EW_THREADS - 1) / EW_THREADS)), dim3(EW_THREADS), 0, s, pre,
                           y_, (int)N);
        return (int)hipGetLastError();
    };
    if (is_vector(1, 256, emb, w->t1)) {   // sinusoid -> linear -> SiLU in one launch
        hipLaunchKernelGGL((gemv_kernel<true, true>), dim3((unsigned)((D + GEMV_WAVES - 1) / GEMV_WAVES)),
                           dim3(64 * GEMV_WAVES), 0, s, nullptr, static_cast<const uint16_t*>(w->t1), h1, (int)D, 256, t);
        LR_LAUNCHED();
    } else {
        hipLaunchKernelGGL(time_sinusoid_kernel, dim3(1), dim3(256), 0, s, t, emb);
        LR_LAUNCHED();
        LR_TRY(linear_silu(emb, w->t1, h1, h1, D, 256));
    }
    LR_TRY(linear_silu(h1, w->t2, temb, ts, D, D));
    LR_TRY(gemm(c, ts, D, w->txt.mod, mod_txt, 6 * D, 1, 6 * D, D, gws, s));
    LR_TRY(gemm(c, ts, D, w->img.mod, mod_img, 6 * D, 1, 6 * D, D, gws, s));

    // attention half: LN + modulation (both streams, one launch), QKV per stream into the joint rows
    hipLaunchKernelGGL(ln_modulate_kernel<false>, dim3((unsigned)S), dim3(LN_THREADS), 0, s, xt, xi, n_txt, (int)D,
                       mod_txt, mod_img, 0, hn, nullptr, 0);
    LR_LAUNCHED();
    const int64_t tD = (int64_t)n_txt * D, tF = (int64_t)n_txt * F;
    LR_TRY(pair_gemm(hn, hn + tD, D, w->txt.qkv, w->img.qkv, qkv, qkv + 3 * tD, 3 * D, 3 * D, D));
    LR_TRY(lr_joint_attention_fused(qkv, qkv + D, qkv + 2 * D, attn, w->q_norm, w->k_norm, LR_TABLE_COSSIN_F32, cos, sin,
                                    cos, sin, 64, LR_PAIR_INTERLEAVED, 128, 1e-6f, (int)S, (int)S, (int)H, (int)H, 0, 0,
                                    1.0f / sqrtf(128.0f), 3 * D, 3 * D, 3 * D, D, 0, ws + L.attn_ws,
                                    lr_joint_attention_workspace_bytes((int)S, (int)H), stream));
    LR_TRY(pair_gemm(attn, attn + tD, D, w->txt.out, w->img.out, hn, hn + tD, D, D, D));
    const unsigned res_blocks = (unsigned)((S * (D / 8) + EW_THREADS - 1) / EW_THREADS);

    // MLP half: the attention half's gated residual (x += gate_0 * hn) and the LayerNorm + modulation in one launch
    hipLaunchKernelGGL(ln_modulate_kernel<true>, dim3((unsigned)S), dim3(LN_THREADS), 0, s, xt, xi, n_txt, (int)D,
                       mod_txt, mod_img, 1, hn, hn, 0);
    LR_LAUNCHED();
    if (n_txt > 0)
        LR_TRY(gemm(c, hn, D, w->txt.mlp_up, big, F, n_txt, F, D, gws, s, false, gelu_fused[0] ? EPI_GELU : EPI_NONE));
    if (n_img > 0)
        LR_TRY(gemm(c, hn + tD, D, w->img.mlp_up, big + tF, F, n_img, F, D, gws, s, false,
                    gelu_fused[1] ? EPI_GELU : EPI_NONE));
    {   // GELU-tanh over the hidden rows whose up-projection did not apply it (text rows first in `big`)
        const int64_t r0 = gelu_fused[0] ? n_txt : 0, r1 = gelu_fused[1] ? n_txt : S;
        const int64_t n8 = (r1 - r0) * F / 8;
        if (n8 > 0) {
            hipLaunchKernelGGL(gelu_tanh_kernel, dim3((unsigned)((n8 + EW_THREADS - 1) / EW_THREADS)), dim3(EW_THREADS),
                               0, s, big + r0 * F, n8);
            LR_LAUNCHED();
        }
    }
    // down-projections, then the MLP half's gated residual: a sliced stream's rows by ksum_residual_kernel (which
    // sums its partials), the other rows by gated_residual_kernel
    float* kpart[2] = {reinterpret_cast<float*>(ws + L.kpart_txt), reinterpret_cast<float*>(ws + L.kpart_img)};
    if (n_txt > 0)
        LR_TRY(gemm(c, big, F, w->txt.mlp_down, ksplit[0] ? (void*)kpart[0] : (void*)attn, D, n_txt, D, F, gws, s, false,
                    ksplit[0] ? EPI_KSPLIT : EPI_NONE));
    if (n_img > 0)
        LR_TRY(gemm(c, big + tF, F, w->img.mlp_down, ksplit[1] ? (void*)kpart[1] : (void*)(attn + tD), D, n_img, D, F,
                    gws, s, false, ksplit[1] ? EPI_KSPLIT : EPI_NONE));
    if (!ksplit[0] && !ksplit[1]) {
        hipLaunchKernelGGL(gated_residual_kernel, dim3(res_blocks), dim3(EW_THREADS), 0, s, xt, xi, n_txt, (int)S,
                           (int)D, attn, mod_txt, mod_img, 1);
        LR_LAUNCHED();
    } else {
        uint16_t* xs[2] = {xt, xi};
        const uint16_t* mods[2] = {mod_txt, mod_img};
        const int64_t rows[2] = {n_txt, n_img}, row0[2] = {0, n_txt};
        for (int k = 0; k < 2; ++k) {
            if (rows[k] == 0) continue;
            const unsigned blocks = (unsigned)((rows[k] * (D / 8) + EW_THREADS - 1) / EW_THREADS);
            if (ksplit[k])
                hipLaunchKernelGGL(ksum_residual_kernel, dim3(blocks), dim3(EW_THREADS), 0, s, xs[k], kpart[k],
                                   (int)rows[k], (int)D, mods[k], 1, KSPLIT);
            else   // this stream's rows alone: gated_residual_kernel with no text rows
                hipLaunchKernelGGL(gated_residual_kernel, dim3(blocks), dim3(EW_THREADS), 0, s, xs[k], xs[k], 0,
                                   (int)rows[k], (int)D, attn + row0[k] * D, mods[k], mods[k], 1);
            LR_LAUNCHED();
        }
    }
#undef LR_LAUNCHED
#undef LR_TRY
    return 0;
}

}  // extern "C"
