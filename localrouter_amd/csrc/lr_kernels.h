// Internal launch interface between the C ABI (lr_abi.hip) and the kernels (attn_fwd.hip, rms_rope.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lr {

// Everything the attention kernel reads, by value (one kernel argument).
struct AttnArgs {
    const uint16_t* q;   // bf16 [W][...] rows, head h at h*128 (+ row stride q_rs)
    const uint16_t* k;   // bf16 keys: key j of kv head g at k + g*k_hs + j*k_rs
    const uint16_t* v;   // bf16 values, same addressing with v_hs / v_rs
    uint16_t* out;       // bf16 [W][...] rows, head h at h*128 (+ row stride o_rs)
    int64_t q_rs, k_rs, v_rs, o_rs;  // row strides (elements)
    int64_t k_hs, v_hs;              // kv-head strides (elements)
    int W, H, HK, G, nkeys, p0, causal;
    float c;                          // scale * log2(e)
    // Fused Q RMSNorm + RoPE (used by the FUSEQ kernels only)
    const float* wq;                  // fp32 [128] norm weight, or null for ones
    int table_kind, pairing, rot;
    const void* qta;                  // table (see TableKind), query row i uses table row i
    const void* qtb;
    int64_t tab_stride;               // table row stride (elements)
    float eps;
    // Split over the keys (plain pipelined kernel, non-causal): nsplit > 1 runs every query block as nsplit workgroups
    // over consecutive key-tile ranges, each writing its unnormalised O (fp32 [H][W][nsplit][128]) and its reference
    // and row sum (fp32 [H][W][nsplit][2], exp2 domain) instead of out; attn_split_combine merges them.
    int nsplit;
    float* part_o;
    float* part_ml;
    // Stream-K launch of the 64-query-per-wave kernel over packed V^T (used when set): 2 SK_MAX_WG slots of
    // SK_SLOT_FLOATS floats, the two parts of each cut block
    float* sk_part;
};

constexpr int SK_MAX_WG = 256;                                   // stream-K workgroups at most (one per CU)
constexpr int SK_SLOT_FLOATS = 4 * (2 * 4 * 16 * 64 + 2 * 2 * 64);   // one part: 4 waves of O, m, l
constexpr size_t SK_AREA_BYTES = (size_t)2 * SK_MAX_WG * SK_SLOT_FLOATS * 4;

// V^T packing of the prepared-keys path: bf16 V rows (key j of kv head g at v + j*v_rs + g*128) into
// [HK][ntiles][128][64], one contiguous 16 KB block of 128 dim rows x 64 keys per 64-key tile, keys past Sk zero.
struct VPackArgs {
    const uint16_t* v;   // null: nothing to pack
    uint16_t* vt;
    int64_t v_rs;
    int Sk, HK, ntiles;
};
constexpr int VT_TILE_KEYS = 64;

// The per-(row, head) RMSNorm + RoPE pass; the same launch also packs vp when vp.v is set (extra blocks).
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
    VPackArgs vp;
};

// Attention tile configurations (queries per wave x waves per workgroup).
enum AttnConfig : int {
    ATTN_CFG_AUTO = 0,
    ATTN_CFG_PIPE_W8 = 1,      // pipelined kernel, 8 waves x 32 queries: 256-query blocks, two waves per SIMD
    ATTN_CFG_PIPE_W4 = 2,      // pipelined kernel, 4 waves x 32 queries: 128-query blocks
    ATTN_CFG_REGSTAGE_W8 = 3,  // register-staged kernel, 8 waves x 32 queries
    ATTN_CFG_PINGPONG_W8 = 4,  // ping-pong kernel: two wave groups alternating MFMA and VALU clusters
    ATTN_CFG_WIDE_W4 = 5,      // pipelined kernel, 4 waves x 64 queries, 32-key tiles: 256-query blocks, one wave per SIMD
    ATTN_CFG_PAIR_W4 = 6,      // pipelined kernel, 4 waves x 64 queries, 64-key tiles, scheduled: 256-query blocks
    ATTN_CFG_WS_W8 = 7,        // warp-specialised kernel: 4 pairs of waves (scores + softmax | PV), 256-query blocks
    ATTN_CFG_PAIR_SK_W4 = 8,   // PAIR_W4 under the stream-K schedule (AttnArgs::sk_part set)
    ATTN_CFG_LAST = 8,
};

// v_t: values come as packed V^T tiles (VPackArgs layout; a.v = the [HK][ntiles] tile array, a.v_hs = ntiles*8192)
// instead of rows; only the pipelined 64-key-tile configurations (AUTO, PIPE_W8, PIPE_W4) read that layout.
hipError_t launch_attention(const AttnArgs& a, bool fuse_q, bool v_t, int config, hipStream_t stream);
// The 64-queries-per-wave kernel (attn_pair.hip): qk = a TableKind (queries normalised and rotated in registers, values
// as packed V^T tiles when v_t) or -1 (plain queries, values as rows).
// keys.hip: gather the kept keys (kmask[j] != 0, in order) and their value rows into kc / vc [n_valid][HK * 128];
// idx: n_valid ints of scratch
hipError_t launch_compact_keys(const void* k, const void* v, int64_t kv_rs, const uint8_t* kmask, int nkeys,
                               int n_valid, int HK, void* idx, void* kc, void* vc, hipStream_t stream);
hipError_t launch_pair(const AttnArgs& a, int qk, bool v_t, hipStream_t stream);
// Merge the key-split partials of a launch with a.nsplit > 1 into out (bf16 rows).
hipError_t launch_split_combine(const AttnArgs& a, hipStream_t stream);
// The warp-specialised kernel (attn_ws.hip): queries fused with table kind qk, values as packed V^T tiles, non-causal.
hipError_t launch_ws(const AttnArgs& a, int qk, hipStream_t stream);
bool attention_config_reads_vt(int config);
hipError_t launch_rms_rope(const RopeArgs& a, hipStream_t stream);
int attention_block_rows(int config);

}  // namespace lr
