// Internal launch interface between the C ABI (lr_abi.hip) and the kernels (attn_fwd.hip, attn_stream.hip,
// kv_image.hip, rms_rope.hip, keys.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lr {

// Everything the attention kernel reads, by value (one kernel argument).
struct AttnArgs {
    const uint16_t* q;   // bf16 [W][...] rows, head h at h*128 (+ row stride q_rs)
    const uint16_t* k;   // bf16 keys: key j of kv head g at k + g*k_hs + j*k_rs
    const uint16_t* v;   // bf16 values, same addressing with v_hs / v_rs (the streaming kernel: rows, v_hs = 128)
    uint16_t* out;       // bf16 [W][...] rows, head h at h*128 (+ row stride o_rs)
    int64_t q_rs, k_rs, v_rs, o_rs;  // row strides (elements)
    int64_t k_hs, v_hs;              // kv-head strides (elements)
    int W, H, HK, G, nkeys, p0, causal;
    float c;                          // scale * log2(e)
    // Split over the keys (plain pipelined kernel, non-causal): nsplit > 1 runs every query block as nsplit workgroups
    // over consecutive key-tile ranges, each writing its unnormalised O (fp32 [H][W][nsplit][128]) and its reference
    // and row sum (fp32 [H][W][nsplit][2], exp2 domain) instead of out; attn_split_combine merges them.
    int nsplit;
    float* part_o;
    float* part_ml;
    // Persistent streaming kernel (attn_stream.hip) with split = 1: the blocks past the last whole round are cut over
    // tail_wg workgroups; the pieces' partials go to `part` (2 slots of STREAM_SLOT_BYTES per workgroup) and their
    // arrivals are counted in `cnt` (one int per cut block, zero between calls). Set by launch_stream.
    int split, tail_wg;
    void* part;
    int* cnt;
};

// The per-(row, head) RMSNorm + RoPE pass.
struct RopeArgs {
    const uint16_t* src;  // bf16, row r head h at src + r*src_rs + h*src_hs
    uint16_t* dst;        // bf16, row r head h at dst + r*dst_rs + h*dst_hs (may equal src: in place)
    int64_t src_rs, src_hs, dst_rs, dst_hs;
    int64_t rows;
    int heads;
    int n_copy;           // leading rows copied unchanged (already normalised and rotated)
    int weight_kind;      // WeightKind
    const void* w;        // [128] fp32 or bf16
    int table_kind, pairing, rot;
    const void* ta;       // row r >= n_copy uses table row r - n_copy
    const void* tb;
    int64_t tab_stride;
    float eps;
    int round_norm;       // 1: round the normalised value to bf16 before the rotation
    float post_scale;     // multiplies the normalised value (before the rotation and the single bf16 rounding)
    int tab_vec;          // 1: cos / sin rows 16-byte aligned (ta, tb and tab_stride), read as 16-byte chunks
};

// Attention configurations (the LR_ATTN_CFG_* values of include/lr_attn.h).
enum AttnConfig : int {
    ATTN_CFG_AUTO = 0,
    ATTN_CFG_PIPE_W8 = 1,      // plain attention, pipelined kernel, 8 waves x 32 queries: 256-query blocks
    ATTN_CFG_PIPE_W4 = 2,      // the same with 4 waves x 32 queries: 128-query blocks, two per CU
    ATTN_CFG_STREAM_W8 = 9,    // fused / prepared calls: the persistent streaming kernel over tile images
};

// Plain attention over value rows (AUTO = PIPE_W8; a.nsplit > 1 splits every query block over the keys).
hipError_t launch_attention(const AttnArgs& a, int config, hipStream_t stream);
// keys.hip: gather the kept keys (kmask[j] != 0, in order) and their value rows into kc / vc [n_valid][HK * 128];
// idx: n_valid ints of scratch
hipError_t launch_compact_keys(const void* k, const void* v, int64_t kv_rs, const uint8_t* kmask, int nkeys,
                               int n_valid, int HK, void* idx, void* kc, void* vc, hipStream_t stream);
// Merge the key-split partials of a launch with a.nsplit > 1 into out (bf16 rows).
hipError_t launch_split_combine(const AttnArgs& a, hipStream_t stream);
hipError_t launch_rms_rope(const RopeArgs& a, hipStream_t stream);

// Keys (RMSNorm + RoPE, rows j < n_pre copied) of a joint-attention call into the tile-image layout of tile_image.h,
// and (copy_v) its values into the workspace as rows (kv_image.hip).
struct KvImageArgs {
    const uint16_t* k;    // bf16 key rows, key j of kv head g at k + j*k_rs + g*128
    const uint16_t* v;    // bf16 value rows, same addressing with v_rs
    int64_t k_rs, v_rs;
    const float* w;       // fp32 [128] key norm weight, or null for ones
    int table_kind, pairing, rot;
    const void* ta;       // key j >= n_pre uses table row j - n_pre
    const void* tb;
    int64_t tab_stride;
    float eps;
    int Sk, HK, n_pre;
    int64_t tiles;        // ceil(Sk / 64)
    void* img_k;          // [HK][tiles] 16 KB key tiles
    void* img_v;          // value rows [tiles * 64][HK][128] (copy_v), else unused
    int copy_v;           // 1: copy the value rows into img_v (rows past Sk zero), for the stage calls
    int* cnt;             // the streaming kernel's arrival counters, zeroed by this launch (ncnt ints; null: none)
    int ncnt;
    int tab_vec;          // as RopeArgs::tab_vec
};
hipError_t launch_kv_image(const KvImageArgs& a, hipStream_t stream);
// The keys / values (as launch_kv_image) and the queries (as launch_rms_rope) of a joint-attention call in one launch;
// both use the same table kind and pairing.
hipError_t launch_joint_prep(const KvImageArgs& kv, const RopeArgs& q, hipStream_t stream);

// The persistent streaming attention kernel (attn_stream.hip): a.k = the key tile images, or with key_rows the key
// rows (bf16, key j of kv head g at a.k + j * a.k_rs + g * a.k_hs, a.k_rs <= STREAM_MAX_V_RS); a.v = the value rows
// (bf16, key j of kv head g at a.v + j * a.v_rs + g * a.v_hs, a.v_rs <= STREAM_MAX_V_RS; rows j < a.nkeys are read);
// a.q = the queries as the attention reads them (bf16 rows with stride a.q_rs; they may be the rows of a.out, which
// each block reads before it overwrites them). nwg = workgroups (at most one per CU).
// Non-causal and causal (p0) calls, any W, H, HK, nkeys.
// a.part / a.cnt: the partial area and arrival counters of the workspace (null: whole blocks only); nwg <=
// STREAM_MAX_WG.
hipError_t launch_stream(const AttnArgs& a, int nwg, hipStream_t stream, bool key_rows = false);
constexpr int64_t STREAM_MAX_V_RS = (int64_t)1 << 24;                   // value row stride (elements) at most
constexpr int STREAM_MAX_WG = 256;                                      // workgroups of one streaming launch at most
constexpr int64_t STREAM_SLOT_BYTES = 8 * (64 * 64 * 4 + 64 * 8);        // one piece's partial: 8 waves' O, m and l
constexpr int64_t STREAM_PART_BYTES = 2 * STREAM_MAX_WG * STREAM_SLOT_BYTES;
constexpr int64_t STREAM_CNT_BYTES = 4 * STREAM_MAX_WG;                 // arrival counters (one per cut block)

}  // namespace lr
