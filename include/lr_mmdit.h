/* The MMDiT double-stream block forward around the joint attention: plain C ABI, gfx950.
 *
 * The reference has no double-stream block (its Qwen engine is the single-stream Qwen 2.1, src/engines/qwen_image/
 * dit.zig:242-308). This block is this library's own definition, in the standard MMDiT form, with the reference's
 * elementwise arithmetic where it has one: the 256-d time sinusoid of kernels/cuda/qwen_image/ops.cu:84-99, the
 * GELU-tanh of ops.cu:48-57 and the gated residual x = fma(a, g, x) of ops.cu:25-31.
 *
 *   emb  = sinusoid(t)                                   [256]   (t in [0, 1], scaled by 1000 as the reference)
 *   temb = silu(emb W_t1^T) W_t2^T                       [D]
 *   mod_s = silu(temb) W_mod_s^T = shift1 | scale1 | gate1 | shift2 | scale2 | gate2, per stream s in {txt, img}
 *   per stream:  h = LayerNorm(x_s) (1 + scale1) + shift1;   qkv_s = h W_qkv_s^T                  [rows_s, 3D]
 *   joint:       rows = txt rows then img rows; per-head QK-RMSNorm (weights q_norm, k_norm) and RoPE (cos/sin
 *                [S, 64] f32, interleaved pairs) fused into the attention: lr_joint_attention_fused_ex
 *   per stream:  x_s += gate1 * (attn_s W_out_s^T)
 *                h = LayerNorm(x_s) (1 + scale2) + shift2;  x_s += gate2 * (gelu_tanh(h W_up_s^T) W_down_s^T)
 *
 * Weights are bf16 row-major [out, in] (torch nn.Linear layout), no biases; LayerNorm without affine, eps 1e-6;
 * activations bf16 between the steps (fp32 inside each kernel and GEMM). The GEMMs are hipBLASLt's (bf16 in and out,
 * fp32 compute); the up-projection carries hipBLASLt's GELU epilogue where an algorithm has it, so its GELU acts on
 * the fp32 product (one bf16 rounding, not two; a shape without such an algorithm runs the library's GELU-tanh
 * kernel on the bf16 product). The down-projection of a stream of at most 1024 rows runs as 4 slices of K into fp32
 * partials, summed in slice order and rounded to bf16 before its gated residual (where hipBLASLt serves the sliced
 * shape; else as one GEMM). Everything else is this library's HIP kernels.
 *
 * Return values follow lr_attn.h: 0 launched, 1 (hipErrorInvalidValue) an argument rejected before any launch, other
 * hipError_t / hipblasStatus_t failures as returned (a hipBLASLt status is reported as 1000 + the status).
 */
#ifndef LR_MMDIT_H
#define LR_MMDIT_H

#include <stddef.h>
#include <stdint.h>

#include "lr_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* One stream's weights (device pointers, bf16 [out, in] row-major). */
typedef struct lr_mmdit_stream_weights {
    const void* mod;      /* [6 D, D]  adaLN modulation */
    const void* qkv;      /* [3 D, D]  q | k | v, heads of 128 in each */
    const void* out;      /* [D, D]    attention output projection */
    const void* mlp_up;   /* [F, D] */
    const void* mlp_down; /* [D, F] */
} lr_mmdit_stream_weights;

typedef struct lr_mmdit_weights {
    const void* t1;       /* [D, 256]  time embedding, first linear */
    const void* t2;       /* [D, D]    time embedding, second linear */
    const float* q_norm;  /* [128] f32 per-head RMSNorm weights of q (both streams) */
    const float* k_norm;  /* [128] f32, of k */
    lr_mmdit_stream_weights txt, img;
} lr_mmdit_weights;

/* A context: the hipBLASLt handle and the GEMM plans of the shapes seen so far (host memory only). *ctx is set on
 * success. Call on the device the blocks will run on. */
int lr_mmdit_create(void** ctx);
int lr_mmdit_destroy(void* ctx);

/* Device scratch one block call needs, bytes (256-aligned); 0 for an unsupported shape (D not a multiple of 128,
 * F not a multiple of 8, sizes <= 0). */
size_t lr_mmdit_workspace_bytes(int n_txt, int n_img, int hidden, int mlp);

/* Build the plans (hipBLASLt's first heuristic result) of the block's row GEMMs for this shape: host work only (no
 * device memory, no synchronisation). The block call needs its shape planned by this call or by lr_mmdit_tune first;
 * it does no planning itself, so it can be recorded under graph capture. Thread-safe per context. */
int lr_mmdit_plan(void* ctx, int n_txt, int n_img, int hidden, int mlp);

/* Optional: time up to `candidates` (<= 16) hipBLASLt heuristic candidates of each of the block's row GEMMs for
 * this shape on the workspace's buffers and keep the fastest (planning the shape as lr_mmdit_plan does).
 * Synchronises the stream and creates events: call it once per shape before timing or capturing blocks. */
int lr_mmdit_tune(void* ctx, const lr_mmdit_weights* w, int n_txt, int n_img, int hidden, int mlp, int candidates,
                  void* workspace, size_t workspace_bytes, lr_stream_t stream);

/* Device scratch of one lr_mmdit_linear_bf16 call, bytes (a block's workspace is larger and also qualifies). */
#define LR_MMDIT_GEMM_WORKSPACE (64u << 20)

/* One linear as the block runs it: y[M, N] (row stride ldy) = x[M, K] (row stride ldx) w[N, K]^T, bf16 in and out,
 * fp32 compute (hipBLASLt), workspace >= LR_MMDIT_GEMM_WORKSPACE bytes. The engines' dense
 * (src/engines/qwen_image/dit.zig:185) on this path; also what bench.py times alone. The first call of a new shape
 * builds its plan (host work); later calls launch only. */
int lr_mmdit_linear_bf16(void* ctx, const void* x, int64_t ldx, const void* w, void* y, int64_t ldy, int M, int N,
                         int K, void* workspace, size_t workspace_bytes, lr_stream_t stream);

/* One block forward, in place on txt [n_txt, D] and img [n_img, D] bf16 (contiguous rows). t: device pointer to one
 * f32 timestep. cos, sin: device [n_txt + n_img, 64] f32 (text rows first). Weights 16-byte aligned. The shape
 * must have been planned (lr_mmdit_plan or lr_mmdit_tune): otherwise it returns hipErrorNotReady (600) and launches
 * nothing. Launches only (no host planning, no synchronisation); calls on one context may come from several threads,
 * each with its own workspace. The workspace's first lr_mmdit_workspace_bytes bytes must not overlap txt, img, t, cos,
 * sin or a weight (rejected before any launch). */
int lr_mmdit_block_bf16(void* ctx, const lr_mmdit_weights* w, void* txt, void* img, int n_txt, int n_img, int hidden,
                        int mlp, const float* t, const float* cos, const float* sin, void* workspace,
                        size_t workspace_bytes, lr_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* LR_MMDIT_H */
