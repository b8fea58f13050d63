// The C ABI (include/lr_attn.h): argument validation, then launches on the caller's stream.
// Like kernels/cuda/minimax/kitchen_launch.cu:193-316 every function checks its arguments before launching and
// returns an int error code. Nothing here synchronises or allocates. The one state kept between calls is that of the
// allocation-free entry point (lr_joint_attention_fused_noalloc): a file-scope static __device__ scratch array
// (LR_JOINT_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends) and a per-device cache of its address, set
// once per device under a mutex (at lr_attn_init, else at the entry point's first call on that device). Calls of that
// entry point that overlap on one GPU share the array and race.
#include <limits.h>
#include <math.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "../../include/lr_attn.h"
#include "lr_common.h"
#include "lr_int8.h"
#include "lr_kernels.h"
#include "tile_image.h"


namespace {

constexpr int ERR_ARGS = (int)hipErrorInvalidValue;

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// A bf16 rows tensor: 16-byte aligned base, row stride a multiple of 8 elements and wide enough for its heads.
inline bool rows_ok(const void* p, int64_t rs, int heads) {
    return p && aligned(p, 16) && rs % 8 == 0 && rs >= (int64_t)heads * lr::D;
}

inline bool scale_ok(float s) { return s > 0.0f && isfinite(s); }

// Key-split count for plain attention over value rows (the pipelined kernel, 256-query blocks): a non-causal launch
// with at most 32 query blocks and at least 16 key tiles is split over the keys into enough ranges of at least 4 key
// tiles to give ~256 workgroups, then merged by a combine pass. 1 = no split (causal calls are never split). Measured
// at 218 queries x 16 / 24 heads the split takes 0.77 / 0.47 / 0.22 of the 128-query pipelined kernel's time at
// 2,000 / 8,000 / 50,220 keys and 1.34 at 600 keys; at 600-1,280 queries the streaming kernel's split tail is faster.
int split_count(int W, int H, int nkeys, int causal) {
    if (causal || W < 1 || H < 1 || nkeys < 1) return 1;
    const int64_t blocks = (int64_t)((W + 255) / 256) * H;
    const int tiles = (nkeys + 63) / 64;
    if (blocks > 32 || tiles < 16) return 1;
    int ns = (int)std::min<int64_t>((256 + blocks - 1) / blocks, tiles / 4);
    ns = std::max(1, std::min(ns, 64));
    const int per = (tiles + ns - 1) / ns;
    return (tiles + per - 1) / per;   // no empty range
}

// Whether a non-causal call over key and value rows that is not key-split runs the streaming kernel (reading key rows
// into tile images in LDS) instead of the pipelined kernels. Measured from 218 to 50,220 queries x 4-32 heads: below
// 4,096 keys the 128-query pipelined kernel is as fast or faster. From 4,096 keys on, with a workspace (its split tail
// cutting the last partial round of blocks over the workgroups) the streaming kernel takes 0.55-0.93 of the pipelined
// kernel's time from 33 query blocks on. Without one it runs whole 256-query blocks (a last partial pass shared by
// the XCDs), and wins when they fill between half a round and a round of the CUs, leave a last round at least half
// full, or fill two rounds or more (432 blocks on 256 CUs: 0.86-0.93 of the 256-query pipelined kernel's time; 800
// and 1,600 blocks with a last round of 32 and 64: 0.98 and 0.94 of the 128-query one's); a few blocks past one round
// (288 blocks: 1.08) favour the pipelined kernel's 128-query blocks.
bool stream_rows(int W, int H, int nkeys, int causal, bool workspace, int cus) {
    if (causal || nkeys < 4096 || cus < 1) return false;
    const int64_t blocks = (int64_t)((W + 255) / 256) * H;
    if (workspace) return blocks > 32;
    const int64_t tail = blocks % cus;
    return blocks <= cus ? 2 * blocks >= cus : blocks >= 2 * (int64_t)cus || tail == 0 || 2 * tail >= cus;
}

// Whether the streaming kernel over key rows cuts the last partial round of blocks over the workgroups (its split
// tail). The pieces of one block stream different key ranges, so blocks of one head no longer share each key tile in
// the caches: at 50,220 keys x 24 heads (617 MB of keys and values) a tail of 216 blocks on 256 CUs ran 1.17-1.23x
// the unsplit time, 144 blocks about the same, 120 blocks 0.78x. Beyond 16,384 keys a tail of three quarters of the
// CUs or more runs unsplit.
bool stream_rows_split(int W, int H, int nkeys, int cus) {
    const int64_t blocks = (int64_t)((W + 255) / 256) * H;
    const int64_t tail = blocks % cus;
    return !(nkeys > 16384 && 4 * tail >= 3 * (int64_t)cus);
}

size_t split_bytes(int W, int H, int ns) {
    if (ns <= 1) return 0;
    const size_t rows = (size_t)H * W * ns;
    return ((rows * lr::D * 4 + 255) & ~(size_t)255) + ((rows * 8 + 255) & ~(size_t)255);
}

int device_cus();

int attention_impl(const void* q, const void* k, const void* v, void* out, int p0, int W, int H, int HK, int nkeys,
                   int causal, float scale, int64_t q_rs, int64_t k_rs, int64_t v_rs, int64_t o_rs, int64_t k_hs,
                   int64_t v_hs, int config, hipStream_t stream, void* workspace = nullptr, size_t ws_bytes = 0) {
    if (W < 1 || H < 1 || HK < 1 || H % HK != 0 || nkeys < 1 || p0 < 0 || (causal != 0 && causal != 1)) return ERR_ARGS;
    if (!scale_ok(scale) || !(config == LR_ATTN_CFG_AUTO || config == LR_ATTN_CFG_PIPE_W8 ||
                              config == LR_ATTN_CFG_PIPE_W4 || config == LR_ATTN_CFG_STREAM_W8))
        return ERR_ARGS;
    if ((int64_t)p0 + W > INT_MAX - 512 || nkeys > INT_MAX - 512 || W > INT_MAX - 512) return ERR_ARGS;
    if (!rows_ok(q, q_rs, H) || !rows_ok(out, o_rs, H)) return ERR_ARGS;
    if (!k || !v || !aligned(k, 16) || !aligned(v, 16) || k_rs % 8 || v_rs % 8 || k_hs % 8 || v_hs % 8) return ERR_ARGS;
    if (k_rs < lr::D || v_rs < lr::D || k_hs < 0 || v_hs < 0) return ERR_ARGS;
    lr::AttnArgs a{};
    a.q = static_cast<const uint16_t*>(q);
    a.k = static_cast<const uint16_t*>(k);
    a.v = static_cast<const uint16_t*>(v);
    a.out = static_cast<uint16_t*>(out);
    a.q_rs = q_rs; a.k_rs = k_rs; a.v_rs = v_rs; a.o_rs = o_rs;
    a.k_hs = k_hs; a.v_hs = v_hs;
    a.W = W; a.H = H; a.HK = HK; a.G = H / HK; a.nkeys = nkeys; a.p0 = p0; a.causal = causal;
    a.c = scale * 1.4426950408889634f;
    const int ns = split_count(W, H, nkeys, causal);
    const bool split = workspace && ns > 1 && (config == LR_ATTN_CFG_AUTO || config == LR_ATTN_CFG_PIPE_W8) &&
                       k_hs == lr::D && v_hs == lr::D && ws_bytes >= split_bytes(W, H, ns) && aligned(workspace, 256);
    if (split) {
        a.nsplit = ns;
        a.part_o = static_cast<float*>(workspace);
        a.part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                             (((size_t)H * W * ns * lr::D * 4 + 255) & ~(size_t)255));
        const hipError_t e = lr::launch_attention(a, LR_ATTN_CFG_PIPE_W8, stream);
        if (e != hipSuccess) return (int)e;
        return (int)lr::launch_split_combine(a, stream);
    }
    const bool ws_split_area = workspace && ws_bytes >= (size_t)LR_JOINT_SPLIT_BYTES && aligned(workspace, 256);
    if (config == LR_ATTN_CFG_AUTO && stream_rows(W, H, nkeys, causal, ws_split_area, device_cus())) {
        config = LR_ATTN_CFG_STREAM_W8;
    } else if (config == LR_ATTN_CFG_AUTO) {
        // 128 queries per workgroup, two workgroups per CU, unless non-causal 256-query blocks fill whole rounds of
        // the CUs: measured at cfg1 / cfg2 / causal GQA shapes W4 takes 0.72 / 0.93 / 0.89 of W8's time, at 12,800
        // and 50,220 tokens the two are within 1.5 %, at 16,384 x 4 heads (exactly one round of 256-query blocks) W8
        // is 2 % faster; causal blocks differ in work, and W4 stays faster there even when the rounds are whole
        const int cus = device_cus();
        const int64_t w8_blocks = (int64_t)((W + 255) / 256) * H;
        config = !causal && cus > 0 && w8_blocks % cus == 0 ? LR_ATTN_CFG_PIPE_W8 : LR_ATTN_CFG_PIPE_W4;
    }
    if (config == LR_ATTN_CFG_STREAM_W8) {
        // the streaming kernel over the key rows: the output's 32-bit buffer range (256 rows * o_rs * 2 bytes < 2^32)
        // and 32-bit per-lane row offsets (k_rs, v_rs <= STREAM_MAX_V_RS); with a workspace, its split tail
        if (o_rs >= ((int64_t)1 << 23) || k_rs > lr::STREAM_MAX_V_RS || v_rs > lr::STREAM_MAX_V_RS) return ERR_ARGS;
        const int cus = std::min(device_cus(), lr::STREAM_MAX_WG);
        if (cus < 1) return (int)hipErrorInvalidDevice;
        if (ws_split_area && stream_rows_split(W, H, nkeys, cus)) {
            a.part = workspace;
            a.cnt = reinterpret_cast<int*>(static_cast<char*>(workspace) + lr::STREAM_PART_BYTES);
        }
        return (int)lr::launch_stream(a, cus, stream, true);
    }
    return (int)lr::launch_attention(a, config, stream);
}

// Table checks shared by the rope entry points. rows_needed: table rows that will be read.
bool table_ok(int kind, const void* ta, const void* tb, int64_t stride, int rot, int pairing, int split_mod) {
    if (kind == LR_TABLE_NONE) return true;
    if (kind < LR_TABLE_NONE || kind > LR_TABLE_MAT2_F32) return false;
    if (rot <= 0 || rot > lr::D || rot % 2) return false;
    if (pairing != LR_PAIR_INTERLEAVED && pairing != LR_PAIR_SPLIT_HALF) return false;
    if (pairing == LR_PAIR_SPLIT_HALF && rot % split_mod) return false;
    if (!ta || stride < 0) return false;
    const int pairs = rot / 2;
    if (kind == LR_TABLE_COSSIN_F32) return tb && aligned(ta, 4) && aligned(tb, 4) && stride >= pairs;
    if (kind == LR_TABLE_MAT2_BF16) return aligned(ta, 8) && stride % 4 == 0 && stride >= 4 * pairs;
    return aligned(ta, 16) && stride % 4 == 0 && stride >= 4 * pairs;  // LR_TABLE_MAT2_F32
}

// Workspace of the fused op and of its two stages: the tile images of the keys (tile_image.h), 16 KB per 64-key tile
// and kv head; then the value area, the same size: value rows [tiles * 64][HK][128] bf16, written by the stage calls
// (the fused call reads the caller's value rows and leaves it unused); then the streaming kernel's split area
// (partials of cut query blocks, then their arrival counters).
static_assert(lr::STREAM_PART_BYTES + lr::STREAM_CNT_BYTES == (int64_t)LR_JOINT_SPLIT_BYTES, "split area size");
size_t ws_bytes_needed(int Sk, int HK) { return 2 * (size_t)lr::img_bytes(Sk, HK) + LR_JOINT_SPLIT_BYTES; }
inline char* split_area(void* ws, int Sk, int HK) { return static_cast<char*>(ws) + 2 * lr::img_bytes(Sk, HK); }

// the configurations of the fused and prepared calls (both the streaming kernel)
inline bool is_stream(int config) { return config == LR_ATTN_CFG_AUTO || config == LR_ATTN_CFG_STREAM_W8; }

// compute units of the current device: the streaming kernel's grid (one workgroup per CU); queried on every call,
// nothing is cached
int device_cus() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    return n;
}

// byte range [lo, hi) of a rows tensor: rows rows of heads heads, row stride rs elements
struct Span {
    uintptr_t lo, hi;
};
inline Span rows_span(const void* p, int64_t rows, int64_t rs, int heads) {
    const uintptr_t lo = reinterpret_cast<uintptr_t>(p);
    return Span{lo, lo + (uintptr_t)(((rows - 1) * rs + (int64_t)heads * lr::D) * 2)};
}
inline Span ws_span(const void* ws, int Sk, int HK) {
    const uintptr_t lo = reinterpret_cast<uintptr_t>(ws);
    return Span{lo, lo + ws_bytes_needed(Sk, HK)};
}
inline bool overlap(Span a, Span b) { return a.lo < b.hi && b.lo < a.hi; }
// byte range of a bf16 [B][X][S][D] tensor with element strides sb, sx, sn (a row's D elements contiguous)
inline Span t4_span(const void* p, int B, int X, int S, int D, int64_t sb, int64_t sx, int64_t sn) {
    const uintptr_t lo = reinterpret_cast<uintptr_t>(p);
    return Span{lo, lo + (uintptr_t)(((int64_t)(B - 1) * sb + (int64_t)(X - 1) * sx + (int64_t)(S - 1) * sn + D) * 2)};
}

// Checks of the keys stage: k_raw and v rows, the key norm weight and table, the workspace.
bool kv_stage_ok(const void* k_raw, int64_t k_rs, const void* v, int64_t v_rs, const float* wk, int table_kind,
                 const void* kta, const void* ktb, int64_t tab_stride, int pairing, int rot, float eps, int Sk, int HK,
                 int n_pre, const void* ws, size_t ws_bytes) {
    if (Sk < 1 || HK < 1 || Sk > INT_MAX - 512 || n_pre < 0 || n_pre > Sk || !(eps >= 0.0f) || !isfinite(eps))
        return false;
    if (!rows_ok(k_raw, k_rs, HK) || !rows_ok(v, v_rs, HK) || (wk && !aligned(wk, 16))) return false;
    if (v_rs > lr::STREAM_MAX_V_RS) return false;   // the attention kernel's 32-bit value-row offsets
    if (Sk > n_pre && !table_ok(table_kind, kta, ktb, tab_stride, rot, pairing, 32)) return false;
    if (!ws || !aligned(ws, 256) || ws_bytes < ws_bytes_needed(Sk, HK)) return false;
    // the launch writes the workspace while it reads the keys and values
    const Span w = ws_span(ws, Sk, HK);
    return !overlap(w, rows_span(k_raw, Sk, k_rs, HK)) && !overlap(w, rows_span(v, Sk, v_rs, HK));
}

// The keys stage (arguments checked): RMSNorm + RoPE of k_raw rows j >= n_pre (k-table row j - n_pre; rows j < n_pre
// copied) and the values, into the workspace's tile images.
// cos / sin tables whose rows are 16-byte aligned are read as 16-byte chunks
inline int tab_vec(int kind, const void* ta, const void* tb, int64_t stride) {
    return kind == LR_TABLE_COSSIN_F32 && aligned(ta, 16) && aligned(tb, 16) && stride % 4 == 0;
}

lr::KvImageArgs kv_args(const void* k_raw, int64_t k_rs, const void* v, int64_t v_rs, const float* wk, int table_kind,
                        const void* kta, const void* ktb, int64_t tab_stride, int pairing, int rot, float eps, int Sk,
                        int HK, int n_pre, void* ws, int copy_v) {
    lr::KvImageArgs r{};
    r.k = static_cast<const uint16_t*>(k_raw);
    r.v = static_cast<const uint16_t*>(v);
    r.k_rs = k_rs; r.v_rs = v_rs;
    r.w = wk;
    r.table_kind = Sk > n_pre ? table_kind : lr::TABLE_NONE; r.pairing = pairing; r.rot = rot;
    r.ta = kta; r.tb = ktb; r.tab_stride = tab_stride; r.eps = eps;
    r.Sk = Sk; r.HK = HK; r.n_pre = n_pre;
    r.tiles = lr::img_tiles(Sk);
    r.img_k = ws;
    r.img_v = static_cast<char*>(ws) + lr::img_bytes(Sk, HK);
    r.copy_v = copy_v;
    r.cnt = reinterpret_cast<int*>(split_area(ws, Sk, HK) + lr::STREAM_PART_BYTES);
    r.ncnt = lr::STREAM_MAX_WG;
    r.tab_vec = tab_vec(r.table_kind, kta, ktb, tab_stride);
    return r;
}
int kv_launch(const void* k_raw, int64_t k_rs, const void* v, int64_t v_rs, const float* wk, int table_kind,
              const void* kta, const void* ktb, int64_t tab_stride, int pairing, int rot, float eps, int Sk, int HK,
              int n_pre, void* ws, hipStream_t stream) {
    return (int)lr::launch_kv_image(
        kv_args(k_raw, k_rs, v, v_rs, wk, table_kind, kta, ktb, tab_stride, pairing, rot, eps, Sk, HK, n_pre, ws, 1),
        stream);
}

// Checks of the query stage: q_raw and q_prep rows (same shape), the table and weight.
bool q_stage_ok(const void* q_raw, int64_t q_rs, const void* q_prep, int64_t p_rs, const float* wq, int table_kind,
                const void* qta, const void* qtb, int64_t tab_stride, int pairing, int rot, float eps, int Sq, int H) {
    if (Sq < 1 || H < 1 || Sq > INT_MAX - 512 || !(eps >= 0.0f) || !isfinite(eps)) return false;
    if (!rows_ok(q_raw, q_rs, H) || !rows_ok(q_prep, p_rs, H) || (wq && !aligned(wq, 16))) return false;
    // in place (the same rows) or apart: each 16-lane group reads its whole row before writing it, nothing else
    if (q_raw != q_prep && overlap(rows_span(q_raw, Sq, q_rs, H), rows_span(q_prep, Sq, p_rs, H))) return false;
    if (q_raw == q_prep && q_rs != p_rs) return false;
    return table_ok(table_kind, qta, qtb, tab_stride, rot, pairing, 32);
}

// The query stage (arguments checked): RMSNorm + RoPE of the q_raw rows into q_prep, rounded once to bf16 as the
// reference's rope_q writes them (rms_rope.hip).
lr::RopeArgs q_args(const void* q_raw, int64_t q_rs, void* q_prep, int64_t p_rs, const float* wq, int table_kind,
                    const void* qta, const void* qtb, int64_t tab_stride, int pairing, int rot, float eps, int Sq,
                    int H) {
    lr::RopeArgs r{};
    r.src = static_cast<const uint16_t*>(q_raw);
    r.dst = static_cast<uint16_t*>(q_prep);
    r.src_rs = q_rs; r.src_hs = lr::D; r.dst_rs = p_rs; r.dst_hs = lr::D;
    r.rows = Sq; r.heads = H; r.n_copy = 0;
    r.weight_kind = wq ? lr::W_F32 : lr::W_NONE; r.w = wq;
    r.table_kind = table_kind; r.pairing = pairing; r.rot = rot;
    r.ta = qta; r.tb = qtb; r.tab_stride = tab_stride;
    r.eps = eps; r.round_norm = 0; r.post_scale = 1.0f;
    r.tab_vec = tab_vec(table_kind, qta, qtb, tab_stride);
    return r;
}
int q_launch(const void* q_raw, int64_t q_rs, void* q_prep, int64_t p_rs, const float* wq, int table_kind,
             const void* qta, const void* qtb, int64_t tab_stride, int pairing, int rot, float eps, int Sq, int H,
             hipStream_t stream) {
    return (int)lr::launch_rms_rope(
        q_args(q_raw, q_rs, q_prep, p_rs, wq, table_kind, qta, qtb, tab_stride, pairing, rot, eps, Sq, H), stream);
}

// Both preparations of the fused call (arguments checked) in one launch; when every key is a prefix key (no key table
// is read) the keys go through their own launch. copy_v: the value rows are copied into the workspace too (the stage
// call lr_joint_prepare, whose workspace must serve lr_joint_attention_images alone; the fused call reads them where
// they are).
int prep_launch(const void* q_raw, int64_t q_rs, void* q_prep, int64_t p_rs, const float* wq, const void* k_raw,
                int64_t k_rs, const void* v, int64_t v_rs, const float* wk, int table_kind, const void* qta,
                const void* qtb, const void* kta, const void* ktb, int64_t tab_stride, int pairing, int rot, float eps,
                int Sq, int Sk, int H, int HK, int n_pre, void* ws, int copy_v, hipStream_t stream) {
    const lr::RopeArgs q = q_args(q_raw, q_rs, q_prep, p_rs, wq, table_kind, qta, qtb, tab_stride, pairing, rot, eps,
                                  Sq, H);
    const lr::KvImageArgs kv = kv_args(k_raw, k_rs, v, v_rs, wk, table_kind, kta, ktb, tab_stride, pairing, rot, eps,
                                       Sk, HK, n_pre, ws, copy_v);
    if (kv.table_kind != q.table_kind) {
        const hipError_t e = lr::launch_kv_image(kv, stream);
        if (e != hipSuccess) return (int)e;
        return (int)lr::launch_rms_rope(q, stream);
    }
    return (int)lr::launch_joint_prep(kv, q, stream);
}

// Checks of the attention stage. o_rs is bounded so that a block's 256 output rows span less than 4 GiB (the
// kernel's 32-bit buffer range: 256 rows * o_rs * 2 bytes < 2^32, i.e. o_rs < 2^23); out must not overlap the
// workspace, and q_prep is either out itself (each block reads its queries before it writes its output over them) or
// apart from it.
bool images_stage_ok(const void* q_prep, int64_t p_rs, const void* ws, size_t ws_bytes, const void* out, int64_t o_rs,
                     int Sq, int Sk, int H, int HK, int p0, int causal, float scale) {
    if (Sq < 1 || Sk < 1 || H < 1 || HK < 1 || H % HK != 0 || p0 < 0 || (causal != 0 && causal != 1)) return false;
    if (!scale_ok(scale)) return false;
    if ((int64_t)p0 + Sq > INT_MAX - 512 || Sk > INT_MAX - 512 || Sq > INT_MAX - 512) return false;
    if (!rows_ok(q_prep, p_rs, H) || !rows_ok(out, o_rs, H) || o_rs >= ((int64_t)1 << 23)) return false;
    if (!ws || !aligned(ws, 256) || ws_bytes < ws_bytes_needed(Sk, HK)) return false;
    const Span so = rows_span(out, Sq, o_rs, H);
    if (overlap(so, ws_span(ws, Sk, HK))) return false;
    if (q_prep == out) return p_rs == o_rs;
    return !overlap(so, rows_span(q_prep, Sq, p_rs, H)) && !overlap(rows_span(q_prep, Sq, p_rs, H), ws_span(ws, Sk, HK));
}

// The attention stage (arguments checked): the persistent streaming kernel, one workgroup per CU (at most
// STREAM_MAX_WG), its last partial round of query blocks cut over all of them (partials and counters in the
// workspace's split area). v / v_rs: the value rows it reads (the caller's, or null for the workspace's value area).
int images_launch(const void* q_prep, int64_t p_rs, const void* ws, void* out, int64_t o_rs, int Sq, int Sk, int H,
                  int HK, int p0, int causal, float scale, hipStream_t stream, const void* v = nullptr,
                  int64_t v_rs = 0) {
    const int cus = std::min(device_cus(), lr::STREAM_MAX_WG);
    if (cus < 1) return (int)hipErrorInvalidDevice;
    lr::AttnArgs a{};
    a.q = static_cast<const uint16_t*>(q_prep);
    a.k = static_cast<const uint16_t*>(ws);
    if (v) {
        a.v = static_cast<const uint16_t*>(v);
        a.v_rs = v_rs;
    } else {
        a.v = reinterpret_cast<const uint16_t*>(static_cast<const char*>(ws) + lr::img_bytes(Sk, HK));
        a.v_rs = (int64_t)HK * lr::D;
    }
    a.out = static_cast<uint16_t*>(out);
    a.q_rs = p_rs; a.o_rs = o_rs;
    a.k_hs = lr::img_tiles(Sk) * (lr::IMG_TILE_BYTES / 2);
    a.v_hs = lr::D;
    a.W = Sq; a.H = H; a.HK = HK; a.G = H / HK; a.nkeys = Sk; a.p0 = p0; a.causal = causal;
    a.c = scale * 1.4426950408889634f;
    char* split = split_area(const_cast<void*>(ws), Sk, HK);
    a.part = split;
    a.cnt = reinterpret_cast<int*>(split + lr::STREAM_PART_BYTES);
    return (int)lr::launch_stream(a, cus, stream);
}

int prepared_impl(const void* q_raw, void* ws, size_t ws_bytes, void* out, const float* wq, int table_kind,
                  const void* qta, const void* qtb, int64_t tab_stride, int pairing, int rot, float eps, int Sq,
                  int Sk, int H, int HK, int p0, int causal, float scale, int64_t q_rs, int64_t o_rs, int config,
                  hipStream_t stream) {
    if (rot == 0) rot = lr::D;
    // the queries are prepared into out's rows, then attended in place there
    if (!is_stream(config) ||
        !q_stage_ok(q_raw, q_rs, out, o_rs, wq, table_kind, qta, qtb, tab_stride, pairing, rot, eps, Sq, H) ||
        !images_stage_ok(out, o_rs, ws, ws_bytes, out, o_rs, Sq, Sk, H, HK, p0, causal, scale))
        return ERR_ARGS;
    const int e = q_launch(q_raw, q_rs, out, o_rs, wq, table_kind, qta, qtb, tab_stride, pairing, rot, eps, Sq, H,
                           stream);
    if (e != 0) return e;
    return images_launch(out, o_rs, ws, out, o_rs, Sq, Sk, H, HK, p0, causal, scale, stream);
}

int fused_impl(const void* q_raw, const void* k_raw, const void* v, void* out, const float* wq, const float* wk,
               int table_kind, const void* qta, const void* qtb, const void* kta, const void* ktb, int64_t tab_stride,
               int pairing, int rot, float eps, int Sq, int Sk, int H, int HK, int p0, int causal, float scale,
               int64_t q_rs, int64_t k_rs, int64_t v_rs, int64_t o_rs, int n_pre, void* ws, size_t ws_bytes,
               int config, hipStream_t stream) {
    // every argument of all three launches is checked before the first one
    if (rot == 0) rot = lr::D;
    if (!is_stream(config) ||
        !q_stage_ok(q_raw, q_rs, out, o_rs, wq, table_kind, qta, qtb, tab_stride, pairing, rot, eps, Sq, H) ||
        !images_stage_ok(out, o_rs, ws, ws_bytes, out, o_rs, Sq, Sk, H, HK, p0, causal, scale) ||
        !kv_stage_ok(k_raw, k_rs, v, v_rs, wk, table_kind, kta, ktb, tab_stride, pairing, rot, eps, Sk, HK, n_pre, ws,
                     ws_bytes))
        return ERR_ARGS;
    // the prepared queries are written into out while the keys and values may still be read, and the preparation
    // writes the workspace while it reads q_raw, k_raw and v: no overlap
    const Span so = rows_span(out, Sq, o_rs, H);
    if (overlap(so, rows_span(k_raw, Sk, k_rs, HK)) || overlap(so, rows_span(v, Sk, v_rs, HK))) return ERR_ARGS;
    if (overlap(rows_span(q_raw, Sq, q_rs, H), ws_span(ws, Sk, HK))) return ERR_ARGS;
    const int e = prep_launch(q_raw, q_rs, out, o_rs, wq, k_raw, k_rs, v, v_rs, wk, table_kind, qta, qtb, kta, ktb,
                              tab_stride, pairing, rot, eps, Sq, Sk, H, HK, n_pre, ws, 0, stream);
    if (e != 0) return e;
    return images_launch(out, o_rs, ws, out, o_rs, Sq, Sk, H, HK, p0, causal, scale, stream, v, v_rs);
}

int rope_impl(const void* src, int64_t src_rs, int64_t src_off, void* dst, int64_t dst_rs, int64_t n, int b,
              int64_t src_bs, int64_t dst_bs, int heads, const void* w, int w_kind, int table_kind, const void* ta,
              const void* tb, int64_t tab_stride, int rot, int pairing, float eps, int round_norm,
              hipStream_t stream) {
    if (rot == 0) rot = lr::D;
    if (n < 1 || b < 1 || heads < 1 || !(eps >= 0.0f) || !isfinite(eps) || (round_norm != 0 && round_norm != 1))
        return ERR_ARGS;
    if (w_kind < LR_WEIGHT_NONE || w_kind > LR_WEIGHT_BF16 || (w_kind != LR_WEIGHT_NONE && !w)) return ERR_ARGS;
    if (w && !aligned(w, 16)) return ERR_ARGS;
    if (!table_ok(table_kind, ta, tb, tab_stride, rot, pairing, 16)) return ERR_ARGS;
    if (!src || !dst || src_off < 0 || src_off % 8 || src_bs % 8 || dst_bs % 8) return ERR_ARGS;
    const char* s0 = static_cast<const char*>(src) + src_off * 2;
    if (!rows_ok(s0, src_rs, heads) || !rows_ok(dst, dst_rs, heads)) return ERR_ARGS;
    if (n > ((int64_t)1 << 40) / heads) return ERR_ARGS;
    for (int bi = 0; bi < b; ++bi) {
        lr::RopeArgs r{};
        r.src = reinterpret_cast<const uint16_t*>(s0) + (int64_t)bi * src_bs;
        r.dst = static_cast<uint16_t*>(dst) + (int64_t)bi * dst_bs;
        r.src_rs = src_rs; r.src_hs = lr::D; r.dst_rs = dst_rs; r.dst_hs = lr::D;
        r.rows = n; r.heads = heads; r.n_copy = 0;
        r.weight_kind = w_kind; r.w = w;
        r.table_kind = table_kind; r.pairing = pairing; r.rot = rot;
        r.ta = ta; r.tb = tb; r.tab_stride = tab_stride;
        r.eps = eps; r.round_norm = round_norm; r.post_scale = 1.0f;
        const hipError_t e = lr::launch_rms_rope(r, stream);
        if (e != hipSuccess) return (int)e;
    }
    return 0;
}

// ------------------------------------------------------------------------------------------------ INT8 chain
// The checks of kitchen_int8_attention_impl (kernels/cuda/minimax/kitchen_launch.cu:199-214): sizes, head dim 64 or
// 128, H % HK, 16-byte aligned bases and strides (a stride whose extent is 1 is never used), a 256-byte aligned
// workspace.
bool i8_sizes_ok(int B, int H, int HK, int Sq, int Sk, int D) {
    if (B < 1 || H < 1 || HK < 1 || Sq < 1 || Sk < 1 || (D != 64 && D != 128) || H % HK != 0) return false;
    if (B > 65535 || H > 65535 || Sq > INT_MAX - 512 || Sk > INT_MAX - 512) return false;
    return (int64_t)((Sq + 255) / 256) * H * B <= INT_MAX;
}

bool i8_tensor_ok(const void* p, int64_t sb, int64_t sh, int64_t sn, int nb, int nh, int nn) {
    auto ok = [](int64_t s, int extent) { return extent < 2 || (s >= 0 && s % 8 == 0); };
    return p && aligned(p, 16) && ok(sb, nb) && ok(sh, nh) && ok(sn, nn);
}

// rope_tab non-null: Kitchen.rmsRope fused into the prep (lr_int8_attention_prep_rope, arguments checked there)
int i8_prep_impl(const void* q, const void* k, const void* v, void* ws, int B, int H, int HK, int Sq, int Sk, int D,
                 int64_t q_sb, int64_t q_sh, int64_t q_sn, int64_t k_sb, int64_t k_sh, int64_t k_sn, int64_t v_sb,
                 int64_t v_sh, int64_t v_sn, hipStream_t stream, const void* rope_tab = nullptr, int64_t tab_rs = 0,
                 const void* qw = nullptr, const void* kw = nullptr, int rot = 0, float eps = 0.0f) {
    if (!i8_sizes_ok(B, H, HK, Sq, Sk, D) || !ws || !aligned(ws, 256)) return ERR_ARGS;
    if (!i8_tensor_ok(q, q_sb, q_sh, q_sn, B, H, Sq) || !i8_tensor_ok(k, k_sb, k_sh, k_sn, B, HK, Sk) ||
        !i8_tensor_ok(v, v_sb, v_sh, v_sn, B, HK, Sk))
        return ERR_ARGS;
    // the prep writes the workspace while it reads q, k, v (and, fused with rmsRope, the table and the norm weights)
    {
        const uintptr_t lo = reinterpret_cast<uintptr_t>(ws);
        const Span w{lo, lo + lr::i8::plan_of(B, H, HK, Sq, Sk, D).total};
        if (overlap(w, t4_span(q, B, H, Sq, D, q_sb, q_sh, q_sn)) ||
            overlap(w, t4_span(k, B, HK, Sk, D, k_sb, k_sh, k_sn)) ||
            overlap(w, t4_span(v, B, HK, Sk, D, v_sb, v_sh, v_sn)))
            return ERR_ARGS;
        if (rope_tab) {
            const uintptr_t t = reinterpret_cast<uintptr_t>(rope_tab);
            const uintptr_t qn = reinterpret_cast<uintptr_t>(qw), kn = reinterpret_cast<uintptr_t>(kw);
            if (overlap(w, Span{t, t + (uintptr_t)(((int64_t)(Sk - 1) * tab_rs + 2 * (int64_t)rot) * 2)}) ||
                overlap(w, Span{qn, qn + 2 * (uintptr_t)D}) || overlap(w, Span{kn, kn + 2 * (uintptr_t)D}))
                return ERR_ARGS;
        }
    }
    lr::i8::PrepArgs a{};
    a.q = static_cast<const uint16_t*>(q);
    a.k = static_cast<const uint16_t*>(k);
    a.v = static_cast<const uint16_t*>(v);
    a.q_sb = q_sb; a.q_sh = q_sh; a.q_sn = q_sn;
    a.k_sb = k_sb; a.k_sh = k_sh; a.k_sn = k_sn;
    a.v_sb = v_sb; a.v_sh = v_sh; a.v_sn = v_sn;
    a.B = B; a.H = H; a.HK = HK; a.Sq = Sq; a.Sk = Sk;
    a.ws = static_cast<uint8_t*>(ws);
    a.p = lr::i8::plan_of(B, H, HK, Sq, Sk, D);
    a.rope_tab = static_cast<const uint16_t*>(rope_tab);
    a.tab_rs = tab_rs;
    a.qw = static_cast<const uint16_t*>(qw);
    a.kw = static_cast<const uint16_t*>(kw);
    a.rope_rot = rot;
    a.rope_eps = eps;
    return (int)lr::i8::launch_prep(a, stream);
}

int i8_kernel_impl(void* out, void* ws, int B, int H, int HK, int Sq, int Sk, int D, float scale, int o_rows,
                   hipStream_t stream) {
    if (!i8_sizes_ok(B, H, HK, Sq, Sk, D) || !ws || !aligned(ws, 256) || !out || !aligned(out, 16)) return ERR_ARGS;
    if (!scale_ok(scale) || (o_rows != 0 && o_rows != 1) || (o_rows && B != 1)) return ERR_ARGS;
    {   // the kernel writes out while it reads the workspace
        const uintptr_t lo = reinterpret_cast<uintptr_t>(ws), o = reinterpret_cast<uintptr_t>(out);
        const Span w{lo, lo + lr::i8::plan_of(B, H, HK, Sq, Sk, D).total};
        if (overlap(w, Span{o, o + (uintptr_t)B * H * Sq * D * 2})) return ERR_ARGS;
    }
    lr::i8::AttnArgs a{};
    a.ws = static_cast<uint8_t*>(ws);
    a.out = static_cast<uint16_t*>(out);
    a.o_sb = (int64_t)H * Sq * D;
    a.o_sh = o_rows ? D : (int64_t)Sq * D;
    a.o_sn = o_rows ? (int64_t)H * D : D;
    a.B = B; a.H = H; a.HK = HK; a.G = H / HK; a.Sq = Sq; a.Sk = Sk;
    a.c = scale * 1.4426950408889634f;
    a.p = lr::i8::plan_of(B, H, HK, Sq, Sk, D);
    return (int)lr::i8::launch_attention(a, device_cus(), stream);
}

int i8_attention_impl(const void* q, const void* k, const void* v, void* out, void* ws, int B, int H, int HK, int Sq,
                      int Sk, int D, int64_t q_sb, int64_t q_sh, int64_t q_sn, int64_t k_sb, int64_t k_sh,
                      int64_t k_sn, int64_t v_sb, int64_t v_sh, int64_t v_sn, float scale, int o_rows,
                      hipStream_t stream) {
    // every argument is checked before the first launch
    if (!i8_sizes_ok(B, H, HK, Sq, Sk, D) || !out || !aligned(out, 16) || !scale_ok(scale) || (o_rows && B != 1))
        return ERR_ARGS;
    {   // out against the workspace (the kernel stage's check) before the prep launches
        const uintptr_t lo = reinterpret_cast<uintptr_t>(ws), o = reinterpret_cast<uintptr_t>(out);
        const Span w{lo, lo + lr::i8::plan_of(B, H, HK, Sq, Sk, D).total};
        if (overlap(w, Span{o, o + (uintptr_t)B * H * Sq * D * 2})) return ERR_ARGS;
    }
    const int e = i8_prep_impl(q, k, v, ws, B, H, HK, Sq, Sk, D, q_sb, q_sh, q_sn, k_sb, k_sh, k_sn, v_sb, v_sh, v_sn,
                               stream);
    if (e != 0) return e;
    return i8_kernel_impl(out, ws, B, H, HK, Sq, Sk, D, scale, o_rows, stream);
}

// ------------------------------------------------------------------------------------------------ no-alloc scratch
// The scratch of lr_joint_attention_fused_noalloc: a file-scope device array (each GPU the library runs on holds its
// own copy until the process ends). Host code never uses the array's name as an address: the per-device address
// comes from hipGetSymbolAddress once per device (at lr_attn_init, else the entry point's first call on the device).
static __device__ __align__(256) uint8_t scratch[LR_JOINT_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::atomic<void*> g_scratch_ptr[MAX_DEVICES];
std::mutex g_scratch_mutex;

// The current device's scratch address (set up on first use); nullptr and *err set when the device cannot be used.
void* device_scratch(int* err) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) { *err = (int)e; return nullptr; }
    if (dev < 0 || dev >= MAX_DEVICES) { *err = (int)hipErrorInvalidDevice; return nullptr; }
    void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (p) return p;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) { *err = e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol; return nullptr; }
        g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
    return p;
}

}  // namespace

extern "C" {

int lr_attn_abi_version(void) { return LR_ATTN_ABI_VERSION; }

int lr_attn_init(void) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return (int)e;
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return (int)hipErrorInvalidDevice;
    int err = 0;
    return device_scratch(&err) ? 0 : err;   // the no-alloc entry point's scratch address on this device
}

int lr_attention_bf16(const void* q, const void* k, const void* v, void* out, int p0, int W, int H, int HK, int nkeys,
                      int causal, float scale, int64_t q_row_stride, int64_t kv_row_stride, int64_t out_row_stride,
                      lr_stream_t stream) {
    if (kv_row_stride < (int64_t)HK * lr::D) return ERR_ARGS;
    return attention_impl(q, k, v, out, p0, W, H, HK, nkeys, causal, scale, q_row_stride, kv_row_stride,
                          kv_row_stride, out_row_stride, lr::D, lr::D, LR_ATTN_CFG_AUTO, stream);
}

size_t lr_attention_ws_bytes(int W, int H, int nkeys, int causal) {
    const int ns = split_count(W, H, nkeys, causal);
    if (ns > 1) return split_bytes(W, H, ns);
    // calls the streaming kernel runs with a workspace: its split tail's partials and arrival counters
    return W >= 1 && H >= 1 && stream_rows(W, H, nkeys, causal, true, 1) ? (size_t)LR_JOINT_SPLIT_BYTES : 0;
}

int lr_attention_bf16_ws(const void* q, const void* k, const void* v, void* out, int p0, int W, int H, int HK,
                         int nkeys, int causal, float scale, int64_t q_row_stride, int64_t kv_row_stride,
                         int64_t out_row_stride, void* workspace, size_t workspace_bytes, lr_stream_t stream) {
    if (kv_row_stride < (int64_t)HK * lr::D) return ERR_ARGS;
    if (workspace_bytes < lr_attention_ws_bytes(W, H, nkeys, causal) || (workspace && !aligned(workspace, 256)))
        return ERR_ARGS;
    if (workspace_bytes > 0 && !workspace) return ERR_ARGS;
    // the call writes partials to the bytes of the workspace it needs while it reads q, k and v and writes out
    const size_t need = lr_attention_ws_bytes(W, H, nkeys, causal);
    if (need > 0 && HK >= 1 && q && k && v && out) {
        const uintptr_t lo = reinterpret_cast<uintptr_t>(workspace);
        const Span w{lo, lo + need};
        if (overlap(w, rows_span(q, W, q_row_stride, H)) || overlap(w, rows_span(k, nkeys, kv_row_stride, HK)) ||
            overlap(w, rows_span(v, nkeys, kv_row_stride, HK)) || overlap(w, rows_span(out, W, out_row_stride, H)))
            return ERR_ARGS;
    }
    return attention_impl(q, k, v, out, p0, W, H, HK, nkeys, causal, scale, q_row_stride, kv_row_stride,
                          kv_row_stride, out_row_stride, lr::D, lr::D, LR_ATTN_CFG_AUTO,
                          reinterpret_cast<hipStream_t>(stream), workspace, workspace_bytes);
}

size_t lr_attention_kmask_workspace_bytes(int n_valid, int HK) {
    if (n_valid < 1 || HK < 1) return 0;
    const size_t idx = ((size_t)n_valid * 4 + 255) & ~(size_t)255;
    const size_t rows = (((size_t)n_valid * HK * lr::D * 2) + 255) & ~(size_t)255;
    return idx + 2 * rows;
}

int lr_attention_kmask_bf16(const void* q, const void* k, const void* v, void* out, const void* kmask, int n_valid,
                            int W, int H, int HK, int nkeys, float scale, int64_t q_row_stride, int64_t kv_row_stride,
                            int64_t out_row_stride, void* workspace, size_t workspace_bytes, lr_stream_t stream) {
    if (!kmask)
        return lr_attention_bf16(q, k, v, out, 0, W, H, HK, nkeys, 0, scale, q_row_stride, kv_row_stride,
                                 out_row_stride, stream);
    const size_t need = lr_attention_kmask_workspace_bytes(n_valid, HK);
    if (n_valid < 1 || n_valid > nkeys || need == 0 || !workspace || workspace_bytes < need ||
        !aligned(workspace, 256))
        return ERR_ARGS;
    if (kv_row_stride < (int64_t)HK * lr::D || kv_row_stride % 8 || !k || !v || !aligned(k, 16) || !aligned(v, 16))
        return ERR_ARGS;
    // the attention's own checks first, against the compacted keys, so that nothing is launched on a bad call
    if (W < 1 || H < 1 || HK < 1 || H % HK != 0 || !scale_ok(scale) || !rows_ok(q, q_row_stride, H) ||
        !rows_ok(out, out_row_stride, H) || W > INT_MAX - 512 || nkeys > INT_MAX - 512)
        return ERR_ARGS;
    // the compaction writes the kept keys' indices, keys and values to the workspace while it reads kmask, k and v,
    // and the attention then reads them beside q and writes out: the workspace's bytes overlap none of those
    {
        const uintptr_t lo = reinterpret_cast<uintptr_t>(workspace), mk = reinterpret_cast<uintptr_t>(kmask);
        const Span w{lo, lo + need};
        if (overlap(w, Span{mk, mk + (uintptr_t)nkeys}) || overlap(w, rows_span(k, nkeys, kv_row_stride, HK)) ||
            overlap(w, rows_span(v, nkeys, kv_row_stride, HK)) || overlap(w, rows_span(q, W, q_row_stride, H)) ||
            overlap(w, rows_span(out, W, out_row_stride, H)))
            return ERR_ARGS;
    }
    char* ws = static_cast<char*>(workspace);
    const size_t idx_bytes = ((size_t)n_valid * 4 + 255) & ~(size_t)255;
    const size_t rows = (((size_t)n_valid * HK * lr::D * 2) + 255) & ~(size_t)255;
    void* kc = ws + idx_bytes;
    void* vc = ws + idx_bytes + rows;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const hipError_t e = lr::launch_compact_keys(k, v, kv_row_stride, static_cast<const uint8_t*>(kmask), nkeys,
                                                 n_valid, HK, ws, kc, vc, s);
    if (e != hipSuccess) return (int)e;
    return lr_attention_bf16(q, kc, vc, out, 0, W, H, HK, n_valid, 0, scale, q_row_stride, (int64_t)HK * lr::D,
                             out_row_stride, stream);
}

int lr_attention_bf16_ex(const void* q, const void* k, const void* v, void* out, int p0, int W, int H, int HK,
                         int nkeys, int causal, float scale, int64_t q_row_stride, int64_t k_row_stride,
                         int64_t v_row_stride, int64_t out_row_stride, int64_t k_head_stride, int64_t v_head_stride,
                         int config, lr_stream_t stream) {
    return attention_impl(q, k, v, out, p0, W, H, HK, nkeys, causal, scale, q_row_stride, k_row_stride, v_row_stride,
                          out_row_stride, k_head_stride, v_head_stride, config, stream);
}

int lr_rms_rope_bf16(const void* src, int64_t src_row_stride, int64_t src_off, void* dst, int64_t dst_row_stride,
                     int64_t n, int b, int64_t src_b_stride, int64_t dst_b_stride, int heads, const void* w, int w_kind,
                     int table_kind, const void* table_a, const void* table_b, int64_t table_row_stride, int rot_dim,
                     int pairing, float eps, int round_norm, lr_stream_t stream) {
    return rope_impl(src, src_row_stride, src_off, dst, dst_row_stride, n, b, src_b_stride, dst_b_stride, heads, w,
                     w_kind, table_kind, table_a, table_b, table_row_stride, rot_dim, pairing, eps, round_norm, stream);
}

int lr_rms_rope_qk_bf16(void* q, void* k, int64_t seq, int heads, int64_t q_row_stride, int64_t k_row_stride,
                        const void* q_norm, const void* k_norm, const void* freqs, int64_t freqs_row_stride,
                        int rot_dim, float eps, lr_stream_t stream) {
    if (!q_norm || !k_norm || !freqs) return ERR_ARGS;
    int e = rope_impl(q, q_row_stride, 0, q, q_row_stride, seq, 1, 0, 0, heads, q_norm, LR_WEIGHT_BF16,
                      LR_TABLE_MAT2_BF16, freqs, nullptr, freqs_row_stride, rot_dim, LR_PAIR_SPLIT_HALF, eps, 1, stream);
    if (e != 0) return e;
    return rope_impl(k, k_row_stride, 0, k, k_row_stride, seq, 1, 0, 0, heads, k_norm, LR_WEIGHT_BF16,
                     LR_TABLE_MAT2_BF16, freqs, nullptr, freqs_row_stride, rot_dim, LR_PAIR_SPLIT_HALF, eps, 1, stream);
}

size_t lr_joint_attention_workspace_bytes(int Sk, int HK) {
    if (Sk < 1 || HK < 1) return 0;
    return ws_bytes_needed(Sk, HK);
}

int lr_joint_attention_fused(const void* q_raw, const void* k_raw, const void* v, void* out, const float* q_norm_w,
                             const float* k_norm_w, int table_kind, const void* q_table_a, const void* q_table_b,
                             const void* k_table_a, const void* k_table_b, int64_t table_row_stride, int pairing,
                             int rot_dim, float eps, int Sq, int Sk, int H, int HK, int p0, int causal, float scale,
                             int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride, int64_t out_row_stride,
                             int n_pre, void* workspace, size_t workspace_bytes, lr_stream_t stream) {
    return fused_impl(q_raw, k_raw, v, out, q_norm_w, k_norm_w, table_kind, q_table_a, q_table_b, k_table_a, k_table_b,
                      table_row_stride, pairing, rot_dim, eps, Sq, Sk, H, HK, p0, causal, scale, q_row_stride,
                      k_row_stride, v_row_stride, out_row_stride, n_pre, workspace, workspace_bytes, LR_ATTN_CFG_AUTO,
                      stream);
}

int lr_joint_kv_prepare(const void* k_raw, int64_t k_row_stride, const void* v, int64_t v_row_stride,
                        const float* k_norm_w, int table_kind, const void* k_table_a, const void* k_table_b,
                        int64_t table_row_stride, int pairing, int rot_dim, float eps, int Sk, int HK, int n_pre,
                        void* workspace, size_t workspace_bytes, lr_stream_t stream) {
    if (rot_dim == 0) rot_dim = lr::D;
    if (!kv_stage_ok(k_raw, k_row_stride, v, v_row_stride, k_norm_w, table_kind, k_table_a, k_table_b,
                     table_row_stride, pairing, rot_dim, eps, Sk, HK, n_pre, workspace, workspace_bytes))
        return ERR_ARGS;
    return kv_launch(k_raw, k_row_stride, v, v_row_stride, k_norm_w, table_kind, k_table_a, k_table_b,
                     table_row_stride, pairing, rot_dim, eps, Sk, HK, n_pre, workspace,
                     reinterpret_cast<hipStream_t>(stream));
}

int lr_joint_attention_prepared(const void* q_raw, void* workspace, size_t workspace_bytes, void* out,
                                const float* q_norm_w, int table_kind, const void* q_table_a, const void* q_table_b,
                                int64_t table_row_stride, int pairing, int rot_dim, float eps, int Sq, int Sk, int H,
                                int HK, int p0, int causal, float scale, int64_t q_row_stride, int64_t out_row_stride,
                                int config, lr_stream_t stream) {
    return prepared_impl(q_raw, workspace, workspace_bytes, out, q_norm_w, table_kind, q_table_a, q_table_b,
                         table_row_stride, pairing, rot_dim, eps, Sq, Sk, H, HK, p0, causal, scale, q_row_stride,
                         out_row_stride, config, reinterpret_cast<hipStream_t>(stream));
}

int lr_joint_q_prepare(const void* q_raw, int64_t q_row_stride, void* q_prep, int64_t q_prep_row_stride,
                       const float* q_norm_w, int table_kind, const void* q_table_a, const void* q_table_b,
                       int64_t table_row_stride, int pairing, int rot_dim, float eps, int Sq, int H,
                       lr_stream_t stream) {
    if (rot_dim == 0) rot_dim = lr::D;
    if (!q_stage_ok(q_raw, q_row_stride, q_prep, q_prep_row_stride, q_norm_w, table_kind, q_table_a, q_table_b,
                    table_row_stride, pairing, rot_dim, eps, Sq, H))
        return ERR_ARGS;
    return q_launch(q_raw, q_row_stride, q_prep, q_prep_row_stride, q_norm_w, table_kind, q_table_a, q_table_b,
                    table_row_stride, pairing, rot_dim, eps, Sq, H, reinterpret_cast<hipStream_t>(stream));
}

int lr_joint_prepare(const void* q_raw, int64_t q_row_stride, void* q_prep, int64_t q_prep_row_stride,
                     const void* k_raw, int64_t k_row_stride, const void* v, int64_t v_row_stride,
                     const float* q_norm_w, const float* k_norm_w, int table_kind, const void* q_table_a,
                     const void* q_table_b, const void* k_table_a, const void* k_table_b, int64_t table_row_stride,
                     int pairing, int rot_dim, float eps, int Sq, int Sk, int H, int HK, int n_pre, void* workspace,
                     size_t workspace_bytes, lr_stream_t stream) {
    if (rot_dim == 0) rot_dim = lr::D;
    if (!q_stage_ok(q_raw, q_row_stride, q_prep, q_prep_row_stride, q_norm_w, table_kind, q_table_a, q_table_b,
                    table_row_stride, pairing, rot_dim, eps, Sq, H) ||
        !kv_stage_ok(k_raw, k_row_stride, v, v_row_stride, k_norm_w, table_kind, k_table_a, k_table_b,
                     table_row_stride, pairing, rot_dim, eps, Sk, HK, n_pre, workspace, workspace_bytes))
        return ERR_ARGS;
    // the prepared queries are written while the keys and values are read; the workspace is written too
    const Span sp = rows_span(q_prep, Sq, q_prep_row_stride, H);
    if (overlap(sp, rows_span(k_raw, Sk, k_row_stride, HK)) || overlap(sp, rows_span(v, Sk, v_row_stride, HK)) ||
        overlap(sp, ws_span(workspace, Sk, HK)) || overlap(rows_span(q_raw, Sq, q_row_stride, H), ws_span(workspace, Sk, HK)))
        return ERR_ARGS;
    return prep_launch(q_raw, q_row_stride, q_prep, q_prep_row_stride, q_norm_w, k_raw, k_row_stride, v, v_row_stride,
                       k_norm_w, table_kind, q_table_a, q_table_b, k_table_a, k_table_b, table_row_stride, pairing,
                       rot_dim, eps, Sq, Sk, H, HK, n_pre, workspace, 1, reinterpret_cast<hipStream_t>(stream));
}

int lr_joint_attention_images(const void* q_prep, int64_t q_prep_row_stride, const void* workspace,
                              size_t workspace_bytes, void* out, int64_t out_row_stride, int Sq, int Sk, int H, int HK,
                              int p0, int causal, float scale, lr_stream_t stream) {
    if (!images_stage_ok(q_prep, q_prep_row_stride, workspace, workspace_bytes, out, out_row_stride, Sq, Sk, H, HK, p0,
                         causal, scale))
        return ERR_ARGS;
    return images_launch(q_prep, q_prep_row_stride, workspace, out, out_row_stride, Sq, Sk, H, HK, p0, causal, scale,
                         reinterpret_cast<hipStream_t>(stream));
}

int lr_joint_attention_fused_ex(const void* q_raw, const void* k_raw, const void* v, void* out, const float* q_norm_w,
                                const float* k_norm_w, int table_kind, const void* q_table_a, const void* q_table_b,
                                const void* k_table_a, const void* k_table_b, int64_t table_row_stride, int pairing,
                                int rot_dim, float eps, int Sq, int Sk, int H, int HK, int p0, int causal, float scale,
                                int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride,
                                int64_t out_row_stride, int n_pre, void* workspace, size_t workspace_bytes, int config,
                                lr_stream_t stream) {
    return fused_impl(q_raw, k_raw, v, out, q_norm_w, k_norm_w, table_kind, q_table_a, q_table_b, k_table_a, k_table_b,
                      table_row_stride, pairing, rot_dim, eps, Sq, Sk, H, HK, p0, causal, scale, q_row_stride,
                      k_row_stride, v_row_stride, out_row_stride, n_pre, workspace, workspace_bytes, config, stream);
}

int lr_joint_attention_fused_noalloc(const void* q_raw, const void* k_raw, const void* v, void* out,
                                     const float* q_norm_w, const float* k_norm_w, int table_kind,
                                     const void* q_table_a, const void* q_table_b, const void* k_table_a,
                                     const void* k_table_b, int64_t table_row_stride, int pairing, int rot_dim,
                                     float eps, int Sq, int Sk, int H, int HK, int p0, int causal, float scale,
                                     int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride,
                                     int64_t out_row_stride, int n_pre, lr_stream_t stream) {
    if (Sk < 1 || HK < 1 || Sk > INT_MAX - 512) return ERR_ARGS;
    const size_t need = ws_bytes_needed(Sk, HK);
    if (need > (size_t)LR_JOINT_NOALLOC_SCRATCH_BYTES) return (int)hipErrorOutOfMemory;
    int err = 0;
    void* ws = device_scratch(&err);
    if (!ws) return err;
    return fused_impl(q_raw, k_raw, v, out, q_norm_w, k_norm_w, table_kind, q_table_a, q_table_b, k_table_a, k_table_b,
                      table_row_stride, pairing, rot_dim, eps, Sq, Sk, H, HK, p0, causal, scale, q_row_stride,
                      k_row_stride, v_row_stride, out_row_stride, n_pre, ws, need, LR_ATTN_CFG_AUTO,
                      reinterpret_cast<hipStream_t>(stream));
}

size_t lr_int8_attention_workspace_bytes(int B, int H, int HK, int Sq, int Sk, int D) {
    if (!i8_sizes_ok(B, H, HK, Sq, Sk, D)) return 0;
    return lr::i8::plan_of(B, H, HK, Sq, Sk, D).total;
}

int lr_int8_attention(const void* q, const void* k, const void* v, void* out, void* workspace, int B, int H, int HK,
                      int Sq, int Sk, int D, int64_t q_sb, int64_t q_sh, int64_t q_sn, int64_t k_sb, int64_t k_sh,
                      int64_t k_sn, int64_t v_sb, int64_t v_sh, int64_t v_sn, float scale, lr_stream_t stream) {
    return i8_attention_impl(q, k, v, out, workspace, B, H, HK, Sq, Sk, D, q_sb, q_sh, q_sn, k_sb, k_sh, k_sn, v_sb,
                             v_sh, v_sn, scale, 0, stream);
}

int lr_int8_attention_rows(const void* q, const void* k, const void* v, void* out, void* workspace, int B, int H,
                           int HK, int Sq, int Sk, int D, int64_t q_sb, int64_t q_sh, int64_t q_sn, int64_t k_sb,
                           int64_t k_sh, int64_t k_sn, int64_t v_sb, int64_t v_sh, int64_t v_sn, float scale,
                           lr_stream_t stream) {
    return i8_attention_impl(q, k, v, out, workspace, B, H, HK, Sq, Sk, D, q_sb, q_sh, q_sn, k_sb, k_sh, k_sn, v_sb,
                             v_sh, v_sn, scale, 1, stream);
}

int lr_int8_attention_prep(const void* q, const void* k, const void* v, void* workspace, int B, int H, int HK, int Sq,
                           int Sk, int D, int64_t q_sb, int64_t q_sh, int64_t q_sn, int64_t k_sb, int64_t k_sh,
                           int64_t k_sn, int64_t v_sb, int64_t v_sh, int64_t v_sn, lr_stream_t stream) {
    return i8_prep_impl(q, k, v, workspace, B, H, HK, Sq, Sk, D, q_sb, q_sh, q_sn, k_sb, k_sh, k_sn, v_sb, v_sh, v_sn,
                        stream);
}

int lr_int8_attention_prep_rope(const void* q, const void* k, const void* v, void* workspace, int B, int H, int HK,
                                int Sq, int Sk, int D, int64_t q_sb, int64_t q_sh, int64_t q_sn, int64_t k_sb,
                                int64_t k_sh, int64_t k_sn, int64_t v_sb, int64_t v_sh, int64_t v_sn,
                                const void* q_norm, const void* k_norm, const void* freqs, int64_t freqs_row_stride,
                                int rot_dim, float eps, lr_stream_t stream) {
    // Kitchen.rmsRope's arguments (lr_rms_rope_qk_bf16): bf16 weights, bf16 [rot/2][2][2] table rows (16-byte
    // aligned: a lane reads its eight pairs as four 16-byte loads), split-half pairs within 16-lane groups
    if (rot_dim == 0) rot_dim = lr::D;
    if (D != 128 || Sq != Sk || rot_dim < 16 || rot_dim > 128 || rot_dim % 16) return ERR_ARGS;
    if (!q_norm || !k_norm || !aligned(q_norm, 16) || !aligned(k_norm, 16) || !(eps >= 0.0f) || !isfinite(eps))
        return ERR_ARGS;
    // (the prep stages a block's 64 table rows by 32-bit offsets from its first row: a row stride up to 2^24)
    if (!freqs || !aligned(freqs, 16) || freqs_row_stride % 8 || freqs_row_stride < 2 * (int64_t)rot_dim ||
        freqs_row_stride > (int64_t)1 << 24)
        return ERR_ARGS;
    return i8_prep_impl(q, k, v, workspace, B, H, HK, Sq, Sk, D, q_sb, q_sh, q_sn, k_sb, k_sh, k_sn, v_sb, v_sh, v_sn,
                        reinterpret_cast<hipStream_t>(stream), freqs, freqs_row_stride, q_norm, k_norm, rot_dim, eps);
}

int lr_int8_attention_kernel(void* out, void* workspace, int B, int H, int HK, int Sq, int Sk, int D,
                             float scale, int o_rows, lr_stream_t stream) {
    return i8_kernel_impl(out, workspace, B, H, HK, Sq, Sk, D, scale, o_rows, stream);
}

}  // extern "C"
