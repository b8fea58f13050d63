/*
 * lr_attn.h -- the C ABI of the MI355X (gfx950) DiT joint-attention path.
 *
 * Every entry point is `extern "C"`, takes plain device pointers, element strides and sizes, launches
 * asynchronously on the caller's stream and returns an int that is a hipError_t:
 *   0 (hipSuccess)             the work was launched;
 *   1 (hipErrorInvalidValue)   an argument was rejected before anything was launched;
 *   any other value            what the HIP runtime reported for the launch.
 * No entry point synchronises, allocates or sets function attributes, so every call may be captured into a HIP graph.
 * Apart from lr_joint_attention_fused_noalloc (one static scratch array per GPU) none keeps mutable global state, and
 * calls on buffers of their own may run concurrently on different streams. The caller owns every buffer.
 *
 * Tensors are bf16 "rows": token-major, heads contiguous, head h of token i at base + i*row_stride + h*128
 * (strides in ELEMENTS). Head dim is 128. Base pointers and row strides must be 16-byte aligned
 * (row strides multiples of 8 elements).
 *
 * The reference interfaces these replace (jayleaton/localrouter):
 *   lr_attention_bf16        <- Ops.attention, src/engines/qwen_image/ops_launch.zig:163-172, which launches
 *                               pattn2_kernel (kernels/cuda/qwen_image/attention.cu:253-444, :816-817)
 *   lr_rms_rope_bf16         <- Triton.ropeRun, src/engines/qwen_image/triton_k.zig:44-53 (tfimage _rms_rope_kernel)
 *   lr_rms_rope_qk_bf16      <- Kitchen.rmsRope, src/engines/minimax_h3/launch.zig:421-441, and
 *                               kitchen_rms_rope_split_half_, kernels/cuda/minimax/kitchen_launch.cu:284-314
 *   lr_joint_attention_fused <- the chain rope_q -> rope_k -> V copy -> attention of Dit.block,
 *                               src/engines/qwen_image/dit.zig:252-293 (and minimax_h3/dit.zig:663-672), as one call;
 *                               its two launches one by one: lr_joint_prepare (rope_k + V copy + rope_q, also
 *                               available as lr_joint_kv_prepare and lr_joint_q_prepare) and
 *                               lr_joint_attention_images (the attention launch, Ops.attention's place)
 *   lr_int8_attention*       <- MiniMax H3's INT8 attention: Kitchen.Plan / attentionPrep / attentionKernel /
 *                               attention, src/engines/minimax_h3/launch.zig:317-419, and kitchen_int8_attention
 *                               {,_rows,_workspace_bytes}, kernels/cuda/minimax/kitchen_launch.cu:193-280
 */
#ifndef LR_ATTN_H
#define LR_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t without pulling in the HIP headers: an opaque pointer (NULL = the default stream). */
typedef struct ihipStream_t* lr_stream_t;

#define LR_ATTN_ABI_VERSION 9
#define LR_HEAD_DIM 128

/* RoPE table kinds: how rotation coefficients are stored per token row, per pair p < rot_dim/2. */
#define LR_TABLE_NONE 0        /* RMSNorm only, no rotation */
#define LR_TABLE_COSSIN_F32 1  /* table_a = cos fp32 [rows][row_stride], table_b = sin fp32, same shape (Qwen-Image) */
#define LR_TABLE_MAT2_BF16 2   /* table_a = bf16 [rows][row_stride] holding [rot/2][2][2] {f00,f01,f10,f11} (H3) */
#define LR_TABLE_MAT2_F32 3    /* as LR_TABLE_MAT2_BF16 in fp32 */
/* A pair (a, b) becomes (f00*a + f01*b, f10*a + f11*b); for COSSIN that is (c*a - s*b, s*a + c*b). */

/* Which dims form a rotated pair. */
#define LR_PAIR_INTERLEAVED 0  /* (2p, 2p+1)        -- Qwen-Image / diffusers, Kandinsky-6 */
#define LR_PAIR_SPLIT_HALF 1   /* (p, p + rot_dim/2) -- MiniMax H3 (comfy-kitchen) */

/* Norm weight element types. */
#define LR_WEIGHT_NONE 0       /* all ones */
#define LR_WEIGHT_F32 1
#define LR_WEIGHT_BF16 2

/* Attention tile configurations for the _ex entry points (0 = the library's choice: LR_ATTN_CFG_STREAM_W8 for the
 * fused and prepared calls; for attention over key and value rows, non-causal calls of at least 4,096 keys run
 * LR_ATTN_CFG_STREAM_W8 over the key rows when their 256-query blocks fill at least half a round of the device's
 * compute units without leaving a last round less than half full, or fill two rounds or more; other calls run
 * LR_ATTN_CFG_PIPE_W4, or LR_ATTN_CFG_PIPE_W8 when non-causal and the 256-query blocks fill whole rounds of the
 * compute units. The workspace call lr_attention_bf16_ws chooses as described there.) */
#define LR_ATTN_CFG_AUTO 0
#define LR_ATTN_CFG_PIPE_W8 1      /* attention over value rows: 256 queries per workgroup (8 waves x 32), direct-to-LDS
                                      K/V ring, next tile's QK^T overlapped with the current tile's softmax */
#define LR_ATTN_CFG_PIPE_W4 2      /* the same kernel with 128 queries per workgroup (4 waves x 32) */
#define LR_ATTN_CFG_STREAM_W8 9    /* one persistent workgroup per CU (8 waves x 32 queries) streaming key tile
                                      images (the LDS image of each 64-key tile, 16 KB: prepared by the fused and
                                      prepared calls, gathered from the key rows by the calls over rows) and value rows
                                      through 4-stage direct-to-LDS rings; softmax against a fixed reference (the
                                      block's first key tile's maximum), query rows whose sums overflowed it recomputed
                                      exactly at the end of the kernel. Over rows it needs out_row_stride < 2^23 and
                                      k / v row strides <= 2^24 elements */

int lr_attn_abi_version(void);

/* Checks that the current HIP device is a gfx950 (MI355X / MI350X) and sets up, once per device, the address of the
 * current device's no-alloc scratch (the static array lr_joint_attention_fused_noalloc uses; its address is looked up
 * with hipGetSymbolAddress and cached per device under a mutex). 0 on success, hipErrorInvalidDevice (101) otherwise,
 * or the error of the address lookup. Optional: lr_joint_attention_fused_noalloc sets the address up at its first
 * call on a device when lr_attn_init was not called there; no other entry point needs it. */
int lr_attn_init(void);

/*
 * Attention over pre-normalised, pre-rotated q/k (drop-in for Ops.attention, ops_launch.zig:163-172).
 *   q   [W][H][128]       row stride q_row_stride
 *   k,v [nkeys][HK][128]  row stride kv_row_stride (both)
 *   out [W][H][128]       row stride out_row_stride
 * out_i = softmax_j(scale * <q_i, k_j>) v_j over j < nkeys, and j <= p0 + i when causal != 0; query head h reads
 * kv head h / (H / HK). Requires W >= 1, nkeys >= 1, H % HK == 0, p0 >= 0, 0 < scale < inf.
 * fp32 accumulation and softmax; P is rounded to bf16 for the PV product; out is rounded to bf16.
 */
int lr_attention_bf16(const void* q, const void* k, const void* v, void* out, int p0, int W, int H, int HK, int nkeys,
                      int causal, float scale, int64_t q_row_stride, int64_t kv_row_stride, int64_t out_row_stride,
                      lr_stream_t stream);

/* lr_attention_bf16 with separate k/v row strides, kv-head strides (k/v head g at base + g*head_stride: 128 for rows,
 * nkeys*128 for head-major [HK][nkeys][128]) and an explicit tile configuration (LR_ATTN_CFG_*). */
int lr_attention_bf16_ex(const void* q, const void* k, const void* v, void* out, int p0, int W, int H, int HK,
                         int nkeys, int causal, float scale, int64_t q_row_stride, int64_t k_row_stride,
                         int64_t v_row_stride, int64_t out_row_stride, int64_t k_head_stride, int64_t v_head_stride,
                         int config, lr_stream_t stream);

/*
 * lr_attention_bf16 with device scratch. A non-causal call with at most 32 blocks of 256 queries x heads and at least
 * 961 keys (16 tiles of 64; e.g. 218 queries over 50,220 keys) is split over the keys into ranges that fill the GPU,
 * each range's partial result written to the workspace, then merged (flash-decoding). Other non-causal calls of at least 4,096 keys
 * run LR_ATTN_CFG_STREAM_W8 over the key rows, whose last partial round of query blocks is cut over all workgroups
 * along the keys, the pieces' partials and arrival counters in the workspace (LR_JOINT_SPLIT_BYTES; the call clears
 * the counters itself). Every other call runs as lr_attention_bf16. lr_attention_ws_bytes is the workspace the call
 * needs (0: none; workspace may then be NULL); those bytes must not overlap q, k, v or out (rejected). Results equal
 * lr_attention_bf16's to fp32 rounding. Calls that overlap on one workspace race.
 */
size_t lr_attention_ws_bytes(int W, int H, int nkeys, int causal);
int lr_attention_bf16_ws(const void* q, const void* k, const void* v, void* out, int p0, int W, int H, int HK,
                         int nkeys, int causal, float scale, int64_t q_row_stride, int64_t kv_row_stride,
                         int64_t out_row_stride, void* workspace, size_t workspace_bytes, lr_stream_t stream);

/*
 * Attention under a key-padding mask: keys j with kmask[j] == 0 are left out (torch's bool key-padding mask, SDPA's
 * additive 0 / -inf), the drop-in for Kandinsky-6's attention.Call with mask = .keys
 * (src/engines/kandinsky6/dit/attention.zig:21-27, dispatched by launch.zig:239-255). Non-causal; q, out rows
 * [W][H*128], k, v rows [nkeys][HK*128] (kv_row_stride for both). kmask: device u8 [nkeys]; n_valid: the number of
 * nonzero bytes, known on the host as the engine's `valid` (1 <= n_valid <= nkeys). The kept keys and value rows are
 * gathered into the workspace, then attended as lr_attention_bf16 does; the workspace's first
 * lr_attention_kmask_workspace_bytes bytes must not overlap kmask, q, k, v or out (rejected). kmask = NULL: no mask
 * (n_valid = nkeys, no workspace needed).
 */
size_t lr_attention_kmask_workspace_bytes(int n_valid, int HK);
int lr_attention_kmask_bf16(const void* q, const void* k, const void* v, void* out, const void* kmask, int n_valid,
                            int W, int H, int HK, int nkeys, float scale, int64_t q_row_stride, int64_t kv_row_stride,
                            int64_t out_row_stride, void* workspace, size_t workspace_bytes, lr_stream_t stream);

/*
 * Per-(token, head) RMSNorm + RoPE of one q/k part, out of place or in place (drop-in for Triton.ropeRun,
 * triton_k.zig:44-53): for batch bi < b, token r < n, head h < heads:
 *   x = src[bi*src_b_stride + r*src_row_stride + src_off + h*128 + d]
 *   y = x / sqrt(mean(x^2) + eps) * w[d]       (fp32; rounded to bf16 here when round_norm != 0)
 *   pairs rotated with table row r; dims >= rot_dim are norm-only
 *   dst[bi*dst_b_stride + r*dst_row_stride + h*128 + d] = bf16(y)
 * w: [128] of w_kind (LR_WEIGHT_*), 16-byte aligned, NULL with LR_WEIGHT_NONE. table_kind LR_TABLE_*, table_row_stride in elements.
 * rot_dim: even, <= 128 (0 = 128); LR_PAIR_SPLIT_HALF needs rot_dim % 16 == 0.
 */
int lr_rms_rope_bf16(const void* src, int64_t src_row_stride, int64_t src_off, void* dst, int64_t dst_row_stride,
                     int64_t n, int b, int64_t src_b_stride, int64_t dst_b_stride, int heads, const void* w, int w_kind,
                     int table_kind, const void* table_a, const void* table_b, int64_t table_row_stride, int rot_dim,
                     int pairing, float eps, int round_norm, lr_stream_t stream);

/*
 * MiniMax H3's fused norm + rotation of q and k in place (drop-in for Kitchen.rmsRope, launch.zig:421-441):
 * q, k [seq][heads][128] with row strides q_row_stride / k_row_stride (packed qkv: both 3*heads*128), bf16 norm
 * weights [128], bf16 freqs [seq][freqs_row_stride] holding [rot_dim/2][2][2], split-half pairs, the normalised value
 * rounded to bf16 before the rotation (rms_rope.cu:143-150). rot_dim 0 = 128.
 */
int lr_rms_rope_qk_bf16(void* q, void* k, int64_t seq, int heads, int64_t q_row_stride, int64_t k_row_stride,
                        const void* q_norm, const void* k_norm, const void* freqs, int64_t freqs_row_stride,
                        int rot_dim, float eps, lr_stream_t stream);

/* The part of the joint attention's workspace behind the key images and value rows: the partial results and arrival
 * counters of query blocks cut over several workgroups (the last, partial round of blocks is spread over all CUs; at
 * most 256 workgroups, two partials of 8 x 16.5 KB each, then 256 int counters). */
#define LR_JOINT_SPLIT_BYTES ((size_t)69207040)

/* Bytes of workspace lr_joint_attention_fused needs: the normalised, rotated keys as [HK][ceil(Sk/64)] tile images of
 * 16 KB (one 64-key tile of one kv head laid out as the attention kernel's LDS holds it; keys past Sk zero), then an
 * area of the same size for value rows, bf16 [ceil(Sk/64) * 64][HK][128] (written by the stage calls
 * lr_joint_kv_prepare / lr_joint_prepare, rows past Sk zero; the fused call reads the caller's v and leaves it
 * unused), then LR_JOINT_SPLIT_BYTES: 2 * HK * ceil(Sk/64) * 16384 + LR_JOINT_SPLIT_BYTES. */
size_t lr_joint_attention_workspace_bytes(int Sk, int HK);

/*
 * The fused joint attention: QK-RMSNorm + RoPE + attention (keys prepared once into the workspace's tile images,
 * queries normalised and rotated into out's rows, which the attention kernel reads before overwriting them; the
 * values are read from v's rows as they are).
 *   q_raw [Sq][H][128], k_raw, v [Sk][HK][128], out [Sq][H][128] bf16 rows with the given row strides
 *   (out_row_stride <= 2^23 elements).
 *   q_norm_w, k_norm_w: fp32 [128], 16-byte aligned, or NULL (ones). eps >= 0.
 *   Query i uses q-table row i; key j >= n_pre uses k-table row j - n_pre; keys j < n_pre are already normalised and
 *   rotated (a cached text prefix) and are used as they are.
 *   table_kind / pairing / rot_dim as in lr_rms_rope_bf16, except LR_PAIR_SPLIT_HALF needs rot_dim % 32 == 0.
 *   Attention as lr_attention_bf16 with nkeys = Sk.
 *   workspace: >= lr_joint_attention_workspace_bytes(Sk, HK) bytes, 256-byte aligned, owned by the caller; its
 *   contents are scratch (clobbered by the call, not read before being written).
 *   out must not overlap the workspace, k_raw or v (q_raw may be out itself: in place).
 */
int lr_joint_attention_fused(const void* q_raw, const void* k_raw, const void* v, void* out, const float* q_norm_w,
                             const float* k_norm_w, int table_kind, const void* q_table_a, const void* q_table_b,
                             const void* k_table_a, const void* k_table_b, int64_t table_row_stride, int pairing,
                             int rot_dim, float eps, int Sq, int Sk, int H, int HK, int p0, int causal, float scale,
                             int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride, int64_t out_row_stride,
                             int n_pre, void* workspace, size_t workspace_bytes, lr_stream_t stream);

/*
 * The two stages of lr_joint_attention_fused as separate calls (same kernels, same results):
 *   lr_joint_kv_prepare         RMSNorm + RoPE of k_raw rows j >= n_pre (k-table row j - n_pre), rows j < n_pre
 *                               copied, into the workspace's key tile images, and the values copied into its
 *                               value rows (so that the workspace alone holds the prepared keys and values);
 *   lr_joint_attention_prepared the attention of q_raw (normalised and rotated into out's rows first) over
 *                               that workspace. config: LR_ATTN_CFG_AUTO or _STREAM_W8.
 * Useful when keys and values are reused (a cached prefix) or to time the stages separately. Several attention calls
 * may share one prepared workspace (its key images and value rows are only read), one after the other: each call
 * also uses the workspace's split area (LR_JOINT_SPLIT_BYTES, left zeroed for the next call), so calls that overlap
 * in time on one workspace race.
 */
int lr_joint_kv_prepare(const void* k_raw, int64_t k_row_stride, const void* v, int64_t v_row_stride,
                        const float* k_norm_w, int table_kind, const void* k_table_a, const void* k_table_b,
                        int64_t table_row_stride, int pairing, int rot_dim, float eps, int Sk, int HK, int n_pre,
                        void* workspace, size_t workspace_bytes, lr_stream_t stream);
int lr_joint_attention_prepared(const void* q_raw, void* workspace, size_t workspace_bytes, void* out,
                                const float* q_norm_w, int table_kind, const void* q_table_a, const void* q_table_b,
                                int64_t table_row_stride, int pairing, int rot_dim, float eps, int Sq, int Sk, int H,
                                int HK, int p0, int causal, float scale, int64_t q_row_stride, int64_t out_row_stride,
                                int config, lr_stream_t stream);

/*
 * The fused op's work as separate calls, in the order of the reference's chain rope_k + V copy -> rope_q -> attention
 * (dit.zig:252-293); lr_joint_attention_fused makes the first two as one launch (lr_joint_prepare, below):
 *   lr_joint_kv_prepare        (above) keys into the workspace's tile images, values into its value rows;
 *   lr_joint_q_prepare         q_raw [Sq][H][128] normalised and rotated (as lr_rms_rope_bf16 with an fp32 weight,
 *                              round_norm 0), rounded once to bf16, into q_prep rows; q_prep may be q_raw itself (in
 *                              place) or out; otherwise it must not overlap q_raw;
 *   lr_joint_attention_images  the attention of those prepared queries over the workspace: one persistent workgroup
 *                              per CU (LR_ATTN_CFG_STREAM_W8). q_prep may be out itself (same row stride: each block
 *                              reads its queries before it writes its output over them); otherwise they must not
 *                              overlap. out_row_stride <= 2^23 elements; out must not overlap the workspace.
 */
int lr_joint_q_prepare(const void* q_raw, int64_t q_row_stride, void* q_prep, int64_t q_prep_row_stride,
                       const float* q_norm_w, int table_kind, const void* q_table_a, const void* q_table_b,
                       int64_t table_row_stride, int pairing, int rot_dim, float eps, int Sq, int H,
                       lr_stream_t stream);
int lr_joint_attention_images(const void* q_prep, int64_t q_prep_row_stride, const void* workspace,
                              size_t workspace_bytes, void* out, int64_t out_row_stride, int Sq, int Sk, int H, int HK,
                              int p0, int causal, float scale, lr_stream_t stream);

/*
 * lr_joint_q_prepare and lr_joint_kv_prepare as one launch: the first of the two launches lr_joint_attention_fused
 * makes (the second is lr_joint_attention_images). Arguments as those two calls, one table kind and pairing for both
 * (each tensor with its own table rows); the same results bit for bit. q_prep must not overlap k_raw, v or the
 * workspace, nor q_raw the workspace.
 */
int lr_joint_prepare(const void* q_raw, int64_t q_row_stride, void* q_prep, int64_t q_prep_row_stride,
                     const void* k_raw, int64_t k_row_stride, const void* v, int64_t v_row_stride,
                     const float* q_norm_w, const float* k_norm_w, int table_kind, const void* q_table_a,
                     const void* q_table_b, const void* k_table_a, const void* k_table_b, int64_t table_row_stride,
                     int pairing, int rot_dim, float eps, int Sq, int Sk, int H, int HK, int n_pre, void* workspace,
                     size_t workspace_bytes, lr_stream_t stream);

/* lr_joint_attention_fused with an explicit tile configuration (LR_ATTN_CFG_*). */
int lr_joint_attention_fused_ex(const void* q_raw, const void* k_raw, const void* v, void* out, const float* q_norm_w,
                                const float* k_norm_w, int table_kind, const void* q_table_a, const void* q_table_b,
                                const void* k_table_a, const void* k_table_b, int64_t table_row_stride, int pairing,
                                int rot_dim, float eps, int Sq, int Sk, int H, int HK, int p0, int causal, float scale,
                                int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride,
                                int64_t out_row_stride, int n_pre, void* workspace, size_t workspace_bytes, int config,
                                lr_stream_t stream);

/*
 * lr_joint_attention_fused without a workspace argument, for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). No counterpart in the reference. The workspace (tile images
 * and split area) lives in a static device array of LR_JOINT_NOALLOC_SCRATCH_BYTES per GPU (held from the library's
 * first use on that GPU until the process ends), so the call allocates nothing: calls with 2 * HK * ceil(Sk/64) *
 * 16384 bytes of images beyond 64 MiB return hipErrorOutOfMemory (2) before launching anything (e.g. HK 24:
 * Sk <= 5440). Every call on one GPU uses that GPU's one array: calls that overlap on a GPU (two streams, two threads)
 * race and must be serialised by the caller; the array keeps the last call's images, which the next call overwrites
 * before reading, and its split area is left zeroed by each call. lr_attn_init sets up the array's address on the
 * current device (else the first call does). Arguments and results as lr_joint_attention_fused.
 */
#define LR_JOINT_NOALLOC_SCRATCH_BYTES (((size_t)64 << 20) + LR_JOINT_SPLIT_BYTES)
int lr_joint_attention_fused_noalloc(const void* q_raw, const void* k_raw, const void* v, void* out,
                                     const float* q_norm_w, const float* k_norm_w, int table_kind,
                                     const void* q_table_a, const void* q_table_b, const void* k_table_a,
                                     const void* k_table_b, int64_t table_row_stride, int pairing, int rot_dim,
                                     float eps, int Sq, int Sk, int H, int HK, int p0, int causal, float scale,
                                     int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride,
                                     int64_t out_row_stride, int n_pre, lr_stream_t stream);

/*
 * MiniMax H3's INT8 attention (the reference's comfy-kitchen SageAttention chain): per kv head a K anchor, Q and K
 * rotated (H4 blocks when Sk <= 256, else the signed H128 / the plain H64) and quantised to int8, V quantised per
 * channel, then out = softmax(scale * Q K^T) V with int8 Q K^T and u8 P x s8 V products (P rounded per key tile of
 * 64 keys, 128 past Sk = 1024 at head dim 128). Arguments as kitchen_int8_attention (kitchen_launch.cu:193-270):
 *   q [B][H][Sq][D], k and v [B][HK][Sk][D] bf16 with element strides (sb, sh, sn) per tensor, last stride 1; each
 *   stride a multiple of 8 elements and each base 16-byte aligned (views into one packed qkv buffer qualify);
 *   D 128 (the engine's, launch.zig:331) or 64 (the wheel's other case, kitchen_launch.cu:196-241: H4 up to 256 keys,
 *   else the plain H64 without the sign flip, 64-key tiles at every length); H a multiple of HK; scale > 0 (the
 *   reference passes D^-0.5 rounded to fp32: 0x3db504f3 for 128);
 *   workspace: lr_int8_attention_workspace_bytes(B, H, HK, Sq, Sk, D) bytes, 256-byte aligned, no initial contents;
 *              those bytes must not overlap q, k, v, out (or, fused with rmsRope, the table and the norm weights):
 *              rejected before any launch.
 * lr_int8_attention writes out bf16 [B][H][Sq][D] contiguous; lr_int8_attention_rows writes rows [Sq][H * D]
 * (B must be 1), the same values. The workspace layout is this library's own (quantised operands, scales, per-tile
 * column sums, a partial area): the prep writes the operands and the kernel reads them. When the query blocks (256
 * rows of a head) leave a last round of at most half the device's compute units, the kernel cuts that round's blocks
 * into up to 4 key ranges and merges them with a second launch, through the workspace's partial area: kernel calls
 * on one workspace must not overlap.
 *   lr_int8_attention_workspace_bytes  <- Kitchen.Plan.of / kitchen_int8_attention_workspace_bytes (0: unsupported)
 *   lr_int8_attention_prep             <- Kitchen.attentionPrep (launch.zig:360-397): anchor, Q/K and V to int8
 *   lr_int8_attention_kernel           <- Kitchen.attentionKernel (launch.zig:399-419); o_rows 0: out [B][H][Sq][D],
 *                                         1: rows [Sq][H * D] (B 1)
 */
size_t lr_int8_attention_workspace_bytes(int B, int H, int HK, int Sq, int Sk, int D);
int lr_int8_attention(const void* q, const void* k, const void* v, void* out, void* workspace, int B, int H, int HK,
                      int Sq, int Sk, int D, int64_t q_sb, int64_t q_sh, int64_t q_sn, int64_t k_sb, int64_t k_sh,
                      int64_t k_sn, int64_t v_sb, int64_t v_sh, int64_t v_sn, float scale, lr_stream_t stream);
int lr_int8_attention_rows(const void* q, const void* k, const void* v, void* out, void* workspace, int B, int H,
                           int HK, int Sq, int Sk, int D, int64_t q_sb, int64_t q_sh, int64_t q_sn, int64_t k_sb,
                           int64_t k_sh, int64_t k_sn, int64_t v_sb, int64_t v_sh, int64_t v_sn, float scale,
                           lr_stream_t stream);
int lr_int8_attention_prep(const void* q, const void* k, const void* v, void* workspace, int B, int H, int HK, int Sq,
                           int Sk, int D, int64_t q_sb, int64_t q_sh, int64_t q_sn, int64_t k_sb, int64_t k_sh,
                           int64_t k_sn, int64_t v_sb, int64_t v_sh, int64_t v_sn, lr_stream_t stream);
int lr_int8_attention_kernel(void* out, void* workspace, int B, int H, int HK, int Sq, int Sk, int D,
                             float scale, int o_rows, lr_stream_t stream);

/*
 * Kitchen.rmsRope fused into Kitchen.attentionPrep: the H3 chain rmsRope -> attentionPrep -> attentionKernel
 * (src/engines/minimax_h3/dit.zig:665-671; the fold the reference names as its next step, docs/dev/RESULTS.md:325-327)
 * as prep_rope -> kernel. The workspace is written exactly as lr_rms_rope_qk_bf16 (in place on q and k) followed by
 * lr_int8_attention_prep would write it -- the same bits -- but q and k are read once and not modified: each row is
 * normalised and rotated in registers, rounded to bf16 as the standalone pass stores it, and quantised.
 *   q, k, v, workspace, strides, B, H, HK, Sq, Sk as lr_int8_attention_prep; D 128; Sq == Sk (token n of q and of k
 *   uses table row n, as in Kitchen.rmsRope over one packed qkv buffer);
 *   q_norm, k_norm, freqs, freqs_row_stride, rot_dim, eps as lr_rms_rope_qk_bf16 (rot_dim 0 = 128, else a multiple of
 *   16); the weights and the table rows 16-byte aligned (freqs_row_stride a multiple of 8 elements, at most 2^24).
 */
int lr_int8_attention_prep_rope(const void* q, const void* k, const void* v, void* workspace, int B, int H, int HK,
                                int Sq, int Sk, int D, int64_t q_sb, int64_t q_sh, int64_t q_sn, int64_t k_sb,
                                int64_t k_sh, int64_t k_sn, int64_t v_sb, int64_t v_sh, int64_t v_sn,
                                const void* q_norm, const void* k_norm, const void* freqs, int64_t freqs_row_stride,
                                int rot_dim, float eps, lr_stream_t stream);


#ifdef __cplusplus
}
#endif

#endif /* LR_ATTN_H */
