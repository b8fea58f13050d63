//! Extern bindings of liblr_attn.so (include/lr_attn.h, include/lr_rope.h, include/lr_mmdit.h) for the engines'
//! HIP build, and the call-site helpers that replace their CUDA launches of the joint-attention path:
//!
//!   attention            <- Ops.attention, src/engines/qwen_image/ops_launch.zig:163-172 (cuda.launch.launch at :171)
//!   ropeRun              <- Triton.ropeRun, src/engines/qwen_image/triton_k.zig:44-53
//!   rmsRope              <- Kitchen.rmsRope, src/engines/minimax_h3/launch.zig:421-441
//!   int8Plan / int8Prep / int8Kernel
//!                        <- Kitchen.Plan / attentionPrep / attentionKernel, src/engines/minimax_h3/launch.zig:317-419
//!   jointAttention       <- the chain rope q -> rope k -> V copy -> attention of Dit.block,
//!                           src/engines/qwen_image/dit.zig:252-293, as one call of two launches
//!
//! Device pointers are u64 as elsewhere in the engines; `Stream` is the HIP stream handle (hipStream_t) that takes
//! cuda.Stream's place. Every entry point returns a hipError_t: 0 launched, 1 (hipErrorInvalidValue) an argument was
//! rejected before anything was launched. Calls are asynchronous on the stream and neither synchronise nor allocate,
//! so they can be recorded into the graphs the engines capture (qwen_image/dit.zig:469-484).

const std = @import("std");

pub const Stream = ?*anyopaque;

pub const HEAD_DIM = 128;
pub const ABI_VERSION: c_int = 9;

pub const TABLE_NONE: c_int = 0;
pub const TABLE_COSSIN_F32: c_int = 1;
pub const TABLE_MAT2_BF16: c_int = 2;
pub const TABLE_MAT2_F32: c_int = 3;
pub const PAIR_INTERLEAVED: c_int = 0;
pub const PAIR_SPLIT_HALF: c_int = 1;
pub const WEIGHT_NONE: c_int = 0;
pub const WEIGHT_F32: c_int = 1;
pub const WEIGHT_BF16: c_int = 2;
pub const CFG_AUTO: c_int = 0;
pub const CFG_PIPE_W8: c_int = 1;
pub const CFG_PIPE_W4: c_int = 2;
pub const CFG_STREAM_W8: c_int = 9;

/// The split area behind the tile images in a joint-attention workspace (LR_JOINT_SPLIT_BYTES).
pub const JOINT_SPLIT_BYTES: usize = 69207040;
/// The no-allocation entry point's static scratch per GPU (LR_JOINT_NOALLOC_SCRATCH_BYTES).
pub const JOINT_NOALLOC_SCRATCH_BYTES: usize = (64 << 20) + JOINT_SPLIT_BYTES;
/// hipBLASLt workspace of one lr_mmdit_linear_bf16 call (LR_MMDIT_GEMM_WORKSPACE).
pub const MMDIT_GEMM_WORKSPACE: usize = 64 << 20;

// ---------------------------------------------------------------------------------------------- include/lr_attn.h
pub extern "lr_attn" fn lr_attn_abi_version() c_int;
pub extern "lr_attn" fn lr_attn_init() c_int;
pub extern "lr_attn" fn lr_attention_bf16(q: u64, k: u64, v: u64, out: u64, p0: c_int, w: c_int, h: c_int, hk: c_int,
    nkeys: c_int, causal: c_int, scale: f32, q_rs: i64, kv_rs: i64, out_rs: i64, s: Stream) c_int;
pub extern "lr_attn" fn lr_attention_bf16_ex(q: u64, k: u64, v: u64, out: u64, p0: c_int, w: c_int, h: c_int, hk: c_int,
    nkeys: c_int, causal: c_int, scale: f32, q_rs: i64, k_rs: i64, v_rs: i64, out_rs: i64, k_hs: i64, v_hs: i64,
    config: c_int, s: Stream) c_int;
pub extern "lr_attn" fn lr_attention_ws_bytes(w: c_int, h: c_int, nkeys: c_int, causal: c_int) usize;
pub extern "lr_attn" fn lr_attention_bf16_ws(q: u64, k: u64, v: u64, out: u64, p0: c_int, w: c_int, h: c_int, hk: c_int,
    nkeys: c_int, causal: c_int, scale: f32, q_rs: i64, kv_rs: i64, out_rs: i64, ws: u64, ws_bytes: usize,
    s: Stream) c_int;
pub extern "lr_attn" fn lr_attention_kmask_workspace_bytes(n_valid: c_int, hk: c_int) usize;
pub extern "lr_attn" fn lr_attention_kmask_bf16(q: u64, k: u64, v: u64, out: u64, kmask: u64, n_valid: c_int, w: c_int,
    h: c_int, hk: c_int, nkeys: c_int, scale: f32, q_rs: i64, kv_rs: i64, out_rs: i64, ws: u64, ws_bytes: usize,
    s: Stream) c_int;
pub extern "lr_attn" fn lr_rms_rope_bf16(src: u64, src_rs: i64, src_off: i64, dst: u64, dst_rs: i64, n: i64, b: c_int,
    src_bs: i64, dst_bs: i64, heads: c_int, w: u64, w_kind: c_int, table_kind: c_int, ta: u64, tb: u64, table_rs: i64,
    rot: c_int, pairing: c_int, eps: f32, round_norm: c_int, s: Stream) c_int;
pub extern "lr_attn" fn lr_rms_rope_qk_bf16(q: u64, k: u64, seq: i64, heads: c_int, q_rs: i64, k_rs: i64, q_norm: u64,
    k_norm: u64, freqs: u64, freqs_rs: i64, rot: c_int, eps: f32, s: Stream) c_int;
pub extern "lr_attn" fn lr_joint_attention_workspace_bytes(sk: c_int, hk: c_int) usize;
pub extern "lr_attn" fn lr_joint_attention_fused(q_raw: u64, k_raw: u64, v: u64, out: u64, q_norm_w: u64, k_norm_w: u64,
    table_kind: c_int, q_ta: u64, q_tb: u64, k_ta: u64, k_tb: u64, table_rs: i64, pairing: c_int, rot: c_int, eps: f32,
    sq: c_int, sk: c_int, h: c_int, hk: c_int, p0: c_int, causal: c_int, scale: f32, q_rs: i64, k_rs: i64, v_rs: i64,
    out_rs: i64, n_pre: c_int, ws: u64, ws_bytes: usize, s: Stream) c_int;
pub extern "lr_attn" fn lr_joint_kv_prepare(k_raw: u64, k_rs: i64, v: u64, v_rs: i64, k_norm_w: u64, table_kind: c_int,
    k_ta: u64, k_tb: u64, table_rs: i64, pairing: c_int, rot: c_int, eps: f32, sk: c_int, hk: c_int, n_pre: c_int,
    ws: u64, ws_bytes: usize, s: Stream) c_int;
pub extern "lr_attn" fn lr_joint_attention_prepared(q_raw: u64, ws: u64, ws_bytes: usize, out: u64, q_norm_w: u64,
    table_kind: c_int, q_ta: u64, q_tb: u64, table_rs: i64, pairing: c_int, rot: c_int, eps: f32, sq: c_int, sk: c_int,
    h: c_int, hk: c_int, p0: c_int, causal: c_int, scale: f32, q_rs: i64, out_rs: i64, config: c_int, s: Stream) c_int;
pub extern "lr_attn" fn lr_joint_q_prepare(q_raw: u64, q_rs: i64, q_prep: u64, p_rs: i64, q_norm_w: u64,
    table_kind: c_int, q_ta: u64, q_tb: u64, table_rs: i64, pairing: c_int, rot: c_int, eps: f32, sq: c_int, h: c_int,
    s: Stream) c_int;
pub extern "lr_attn" fn lr_joint_attention_images(q_prep: u64, p_rs: i64, ws: u64, ws_bytes: usize, out: u64,
    out_rs: i64, sq: c_int, sk: c_int, h: c_int, hk: c_int, p0: c_int, causal: c_int, scale: f32, s: Stream) c_int;
pub extern "lr_attn" fn lr_joint_prepare(q_raw: u64, q_rs: i64, q_prep: u64, p_rs: i64, k_raw: u64, k_rs: i64, v: u64,
    v_rs: i64, q_norm_w: u64, k_norm_w: u64, table_kind: c_int, q_ta: u64, q_tb: u64, k_ta: u64, k_tb: u64,
    table_rs: i64, pairing: c_int, rot: c_int, eps: f32, sq: c_int, sk: c_int, h: c_int, hk: c_int, n_pre: c_int,
    ws: u64, ws_bytes: usize, s: Stream) c_int;
pub extern "lr_attn" fn lr_joint_attention_fused_ex(q_raw: u64, k_raw: u64, v: u64, out: u64, q_norm_w: u64,
    k_norm_w: u64, table_kind: c_int, q_ta: u64, q_tb: u64, k_ta: u64, k_tb: u64, table_rs: i64, pairing: c_int,
    rot: c_int, eps: f32, sq: c_int, sk: c_int, h: c_int, hk: c_int, p0: c_int, causal: c_int, scale: f32, q_rs: i64,
    k_rs: i64, v_rs: i64, out_rs: i64, n_pre: c_int, ws: u64, ws_bytes: usize, config: c_int, s: Stream) c_int;
pub extern "lr_attn" fn lr_joint_attention_fused_noalloc(q_raw: u64, k_raw: u64, v: u64, out: u64, q_norm_w: u64,
    k_norm_w: u64, table_kind: c_int, q_ta: u64, q_tb: u64, k_ta: u64, k_tb: u64, table_rs: i64, pairing: c_int,
    rot: c_int, eps: f32, sq: c_int, sk: c_int, h: c_int, hk: c_int, p0: c_int, causal: c_int, scale: f32, q_rs: i64,
    k_rs: i64, v_rs: i64, out_rs: i64, n_pre: c_int, s: Stream) c_int;
pub extern "lr_attn" fn lr_int8_attention_workspace_bytes(b: c_int, h: c_int, hk: c_int, sq: c_int, sk: c_int,
    d: c_int) usize;
pub extern "lr_attn" fn lr_int8_attention(q: u64, k: u64, v: u64, out: u64, ws: u64, b: c_int, h: c_int, hk: c_int,
    sq: c_int, sk: c_int, d: c_int, q_sb: i64, q_sh: i64, q_sn: i64, k_sb: i64, k_sh: i64, k_sn: i64, v_sb: i64,
    v_sh: i64, v_sn: i64, scale: f32, s: Stream) c_int;
pub extern "lr_attn" fn lr_int8_attention_rows(q: u64, k: u64, v: u64, out: u64, ws: u64, b: c_int, h: c_int, hk: c_int,
    sq: c_int, sk: c_int, d: c_int, q_sb: i64, q_sh: i64, q_sn: i64, k_sb: i64, k_sh: i64, k_sn: i64, v_sb: i64,
    v_sh: i64, v_sn: i64, scale: f32, s: Stream) c_int;
pub extern "lr_attn" fn lr_int8_attention_prep(q: u64, k: u64, v: u64, ws: u64, b: c_int, h: c_int, hk: c_int, sq: c_int,
    sk: c_int, d: c_int, q_sb: i64, q_sh: i64, q_sn: i64, k_sb: i64, k_sh: i64, k_sn: i64, v_sb: i64, v_sh: i64,
    v_sn: i64, s: Stream) c_int;
pub extern "lr_attn" fn lr_int8_attention_kernel(out: u64, ws: u64, b: c_int, h: c_int, hk: c_int, sq: c_int, sk: c_int,
    d: c_int, scale: f32, o_rows: c_int, s: Stream) c_int;
pub extern "lr_attn" fn lr_int8_attention_prep_rope(q: u64, k: u64, v: u64, ws: u64, b: c_int, h: c_int, hk: c_int,
    sq: c_int, sk: c_int, d: c_int, q_sb: i64, q_sh: i64, q_sn: i64, k_sb: i64, k_sh: i64, k_sn: i64, v_sb: i64,
    v_sh: i64, v_sn: i64, q_norm: u64, k_norm: u64, freqs: u64, freqs_row_stride: i64, rot_dim: c_int, eps: f32,
    s: Stream) c_int;

// ---------------------------------------------------------------------------------------------- include/lr_rope.h
pub extern "lr_attn" fn lr_rope_sincos(x: [*]const f64, n: i64, sin_out: [*]f64, cos_out: [*]f64) c_int;
pub extern "lr_attn" fn lr_rope_qwen_omegas(out: *[64]f64) void;
pub extern "lr_attn" fn lr_rope_qwen_text_ids(ids: [*]f32, n: c_int, first: c_int) c_int;
pub extern "lr_attn" fn lr_rope_qwen_image_ids(ids: [*]f32, h: c_int, w: c_int, pos: c_int, target_h: c_int,
    target_w: c_int) c_int;
pub extern "lr_attn" fn lr_rope_qwen_table(ids: [*]const f32, n: c_int, omegas: ?[*]const f64, cos_out: [*]f32,
    sin_out: [*]f32) c_int;
pub extern "lr_attn" fn lr_rope_grid2d_table(n_text: c_int, gh: c_int, gw: c_int, theta: f64, cos_out: [*]f32,
    sin_out: [*]f32) c_int;
pub extern "lr_attn" fn lr_rope_edit_table(n_text: c_int, frames: c_int, gh: c_int, gw: c_int, cos_out: [*]f32,
    sin_out: [*]f32) c_int;
pub extern "lr_attn" fn lr_rope_video3d_table(n_text: c_int, t: c_int, gh: c_int, gw: c_int, theta: f64,
    cos_out: [*]f32, sin_out: [*]f32) c_int;
pub extern "lr_attn" fn lr_rope_h3_rows(l: c_int, t: c_int, h: c_int, w: c_int, a: c_int, first_frame: c_int) i64;
pub extern "lr_attn" fn lr_rope_h3_positions(l: c_int, t: c_int, h: c_int, w: c_int, a: c_int, first_frame: c_int,
    pos: [*][3]f64) c_int;
pub extern "lr_attn" fn lr_rope_h3_table(pos: [*]const [3]f64, rows: i64, inv_freq: *const [16]f32, out: [*]u16) c_int;

// ---------------------------------------------------------------------------------------------- include/lr_mmdit.h
pub const MmditStream = extern struct { mod: u64, qkv: u64, out: u64, mlp_up: u64, mlp_down: u64 };
pub const MmditWeights = extern struct { t1: u64, t2: u64, q_norm: u64, k_norm: u64, txt: MmditStream, img: MmditStream };
pub extern "lr_attn" fn lr_mmdit_create(ctx: *?*anyopaque) c_int;
pub extern "lr_attn" fn lr_mmdit_destroy(ctx: ?*anyopaque) c_int;
pub extern "lr_attn" fn lr_mmdit_workspace_bytes(n_txt: c_int, n_img: c_int, hidden: c_int, mlp: c_int) usize;
pub extern "lr_attn" fn lr_mmdit_plan(ctx: ?*anyopaque, n_txt: c_int, n_img: c_int, hidden: c_int, mlp: c_int) c_int;
pub extern "lr_attn" fn lr_mmdit_tune(ctx: ?*anyopaque, w: *const MmditWeights, n_txt: c_int, n_img: c_int,
    hidden: c_int, mlp: c_int, candidates: c_int, ws: u64, ws_bytes: usize, s: Stream) c_int;
pub extern "lr_attn" fn lr_mmdit_linear_bf16(ctx: ?*anyopaque, x: u64, ldx: i64, w: u64, y: u64, ldy: i64, m: c_int,
    n: c_int, k: c_int, ws: u64, ws_bytes: usize, s: Stream) c_int;
pub extern "lr_attn" fn lr_mmdit_block_bf16(ctx: ?*anyopaque, w: *const MmditWeights, txt: u64, img: u64, n_txt: c_int,
    n_img: c_int, hidden: c_int, mlp: c_int, t: u64, cos: u64, sin: u64, ws: u64, ws_bytes: usize, s: Stream) c_int;

// ---------------------------------------------------------------------------------------------- errors
pub const Error = error{ LrInvalidArgument, LrNotReady, LrOutOfMemory, LrLaunch };

/// A returned hipError_t as a Zig error: 1 rejected argument (nothing launched), 2 the no-allocation scratch is too
/// small, 600 an MMDiT shape not planned yet, anything else a HIP launch error.
pub fn check(rc: c_int) Error!void {
    return switch (rc) {
        0 => {},
        1 => error.LrInvalidArgument,
        2 => error.LrOutOfMemory,
        600 => error.LrNotReady,
        else => error.LrLaunch,
    };
}

// ---------------------------------------------------------------------------------------------- call-site helpers
/// f32(1 / sqrt(128)) = 0x3DB504F3, the scale Ops.attention passes (ops_launch.zig:163-172).
pub const SCALE_128: f32 = @bitCast(@as(u32, 0x3db504f3));

/// Ops.attention: q / out rows [w, heads, 128], k / v rows [nkeys, kv_heads, 128]; causal query i sits at p0 + i.
pub fn attention(s: Stream, q: u64, k: u64, v: u64, out: u64, w: u32, heads: u32, kv_heads: u32, nkeys: u32,
    causal: bool, p0: u32) Error!void {
    const row: i64 = @as(i64, heads) * HEAD_DIM;
    const kv_row: i64 = @as(i64, kv_heads) * HEAD_DIM;
    try check(lr_attention_bf16(q, k, v, out, @intCast(p0), @intCast(w), @intCast(heads), @intCast(kv_heads),
        @intCast(nkeys), @intFromBool(causal), SCALE_128, row, kv_row, row, s));
}

/// Triton.ropeRun's Rope{} (triton_k.zig:44-53): fp32 weight [128], fp32 cos / sin [n, 64], 32 heads.
pub const Rope = struct {
    src: u64,
    w: u64,
    cos: u64,
    sin: u64,
    dst: u64,
    src_b_stride: i64,
    src_row_stride: i64,
    src_off: i64,
    dst_b_stride: i64,
    dst_row_stride: i64,
    n: i64,
    b: u32,
};

pub fn ropeRun(s: Stream, r: Rope, eps: f32) Error!void {
    try check(lr_rms_rope_bf16(r.src, r.src_row_stride, r.src_off, r.dst, r.dst_row_stride, r.n, @intCast(r.b),
        r.src_b_stride, r.dst_b_stride, 32, r.w, WEIGHT_F32, TABLE_COSSIN_F32, r.cos, r.sin, 64, 128,
        PAIR_INTERLEAVED, eps, 0, s));
}

/// Kitchen.rmsRope: in place on packed qkv [seq, 3 heads 128] (q at element 0, k at heads 128), bf16 weights, bf16
/// table [seq, rot/2, 2, 2], split-half pairs, the normalised value rounded before the rotation.
pub fn rmsRope(s: Stream, qkv: u64, freqs: u64, qw: u64, kw: u64, heads: u32, seq: u32, rot: u32, eps: f32) Error!void {
    const row: i64 = 3 * @as(i64, heads) * HEAD_DIM;
    try check(lr_rms_rope_qk_bf16(qkv, qkv + @as(u64, heads) * HEAD_DIM * 2, seq, @intCast(heads), row, row, qw, kw,
        freqs, @as(i64, rot) * 2, @intCast(rot), eps, s));
}

/// Kitchen.Plan.of(heads, seq).total: the INT8 chain's workspace bytes (the layout is the library's own).
pub fn int8Plan(heads: u32, seq: u32) usize {
    return lr_int8_attention_workspace_bytes(1, @intCast(heads), @intCast(heads), @intCast(seq), @intCast(seq),
        HEAD_DIM);
}

/// Kitchen.attentionPrep on one packed qkv buffer.
pub fn int8Prep(s: Stream, qkv: u64, ws: u64, heads: u32, seq: u32) Error!void {
    const row: i64 = 3 * @as(i64, heads) * HEAD_DIM;
    const sb: i64 = @as(i64, seq) * row;
    const h2: u64 = @as(u64, heads) * HEAD_DIM * 2;
    try check(lr_int8_attention_prep(qkv, qkv + h2, qkv + 2 * h2, ws, 1, @intCast(heads), @intCast(heads),
        @intCast(seq), @intCast(seq), HEAD_DIM, sb, HEAD_DIM, row, sb, HEAD_DIM, row, sb, HEAD_DIM, row, s));
}

/// Kitchen.rmsRope + Kitchen.attentionPrep as one launch pair on one packed qkv buffer (dit.zig:665-668): q and k are
/// normalised and rotated while they are quantised, and left unmodified in qkv; the workspace holds the same bits as
/// after rmsRope (in place) then attentionPrep.
pub fn int8PrepRope(s: Stream, qkv: u64, ws: u64, freqs: u64, qw: u64, kw: u64, heads: u32, seq: u32, rot: u32,
    eps: f32) Error!void {
    const row: i64 = 3 * @as(i64, heads) * HEAD_DIM;
    const sb: i64 = @as(i64, seq) * row;
    const h2: u64 = @as(u64, heads) * HEAD_DIM * 2;
    try check(lr_int8_attention_prep_rope(qkv, qkv + h2, qkv + 2 * h2, ws, 1, @intCast(heads), @intCast(heads),
        @intCast(seq), @intCast(seq), HEAD_DIM, sb, HEAD_DIM, row, sb, HEAD_DIM, row, sb, HEAD_DIM, row, qw, kw, freqs,
        @as(i64, rot) * 2, @intCast(rot), eps, s));
}

/// Kitchen.attentionKernel: out [heads, seq, 128], or rows [seq, heads 128] when `rows`.
pub fn int8Kernel(s: Stream, out: u64, ws: u64, heads: u32, seq: u32, rows: bool) Error!void {
    try check(lr_int8_attention_kernel(out, ws, 1, @intCast(heads), @intCast(heads), @intCast(seq), @intCast(seq),
        HEAD_DIM, SCALE_128, @intFromBool(rows), s));
}

/// Dit.block's chain (dit.zig:252-293) as one call. q: the queries in packed qkv [n, 3 heads 128]; kbuf / vbuf: rows
/// [n_pre + n, heads 128], the cached prefix (keys already normalised and rotated, dit.zig:494) followed by this
/// step's raw keys and values (copied out of qkv as the engine copies V today, dit.zig:258-263). q and k are
/// normalised (fp32 weights) and rotated (fp32 cos / sin [*, 64]; query i row i, key j >= n_pre row j - n_pre), then
/// attended over the n_pre + n keys into out rows [n, heads 128]. ws: at least
/// lr_joint_attention_workspace_bytes(n_pre + n, heads) bytes, 256-byte aligned, from the engine's arena.
pub fn jointAttention(s: Stream, qkv: u64, kbuf: u64, vbuf: u64, out: u64, q_norm: u64, k_norm: u64, q_cos: u64,
    q_sin: u64, k_cos: u64, k_sin: u64, heads: u32, n: u32, n_pre: u32, ws: u64, ws_bytes: usize, eps: f32) Error!void {
    const qkv_row: i64 = 3 * @as(i64, heads) * HEAD_DIM;
    const row: i64 = @as(i64, heads) * HEAD_DIM;
    const sk: u32 = n_pre + n;
    try check(lr_joint_attention_fused(qkv, kbuf, vbuf, out, q_norm, k_norm, TABLE_COSSIN_F32, q_cos, q_sin, k_cos,
        k_sin, 64, PAIR_INTERLEAVED, 128, eps, @intCast(n), @intCast(sk), @intCast(heads), @intCast(heads), 0, 0,
        SCALE_128, qkv_row, row, row, row, @intCast(n_pre), ws, ws_bytes, s));
}

test "hipError_t mapping" {
    try check(0);
    try std.testing.expectError(error.LrInvalidArgument, check(1));
    try std.testing.expectError(error.LrOutOfMemory, check(2));
    try std.testing.expectError(error.LrNotReady, check(600));
    try std.testing.expectError(error.LrLaunch, check(719));
}

test "constants of the C headers" {
    try std.testing.expectEqual(@as(u32, 0x3db504f3), @as(u32, @bitCast(SCALE_128)));
    try std.testing.expectEqual(@as(usize, 2 * 256 * 8 * (64 * 64 * 4 + 64 * 8) + 4 * 256), JOINT_SPLIT_BYTES);
    try std.testing.expectEqual(@as(usize, 14 * 8), @sizeOf(MmditWeights));   // lr_mmdit_weights: 14 pointers
}
