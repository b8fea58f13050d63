// The INT8 attention chain (MiniMax H3's quantised attention): workspace plan and launch interface between the C
// ABI (lr_abi.hip) and the kernels (int8_attn.hip).
//
// The chain follows src/engines/minimax_h3/launch.zig:317-419 (Kitchen.Plan / attentionPrep / attentionKernel) and
// kernels/cuda/minimax/kitchen_launch.cu:193-280: a K anchor per kv head, Q and K rotated (H4 when Sk <= 256, else
// the signed H128 at head dim 128 or the plain H64 at head dim 64) and quantised to int8, V quantised per channel,
// then softmax(scale Q K^T) V with int8 QK^T and u8 P x s8 V products. Head dim D is 128 (the engine's) or 64 (the
// wheel's other case). The workspace layout is this library's own, laid out for the gfx950 kernels:
//   q8     int8 [B][H][Sq][D]                       rotated queries, plain rows
//   k8     int8 [B][HK][skp][D]                     rotated keys minus the anchor; 16-byte chunk c of key row r stored at
//                                                   c ^ k_swz(r, D); rows past Sk (skp = ntiles * cta) repeat real keys
//                                                   (see quant_k), so that their scores never raise a row max
//   vt     int8 [B][HK][ntiles][D][cta]             V^T tiles; chunk c of dim row d at c ^ v_swz(d), keys past Sk zero
//   aux    [B][HK][ntiles] blocks of 1 KB           per tile: int16 column sums of vt over each half tile, laid out
//                                                   [half][lane 0..31][dim block 0..D/32-1] (dim = 32 * block + lane),
//                                                   then the tile's K scales as fp32 [half][block] (key block b, half
//                                                   h -> scale of keys 32 b + 16 h .. + 15)
//   qs     fp32 [B][H][Sq]                          one scale per query row
//   vs     fp32 [B][HK][D]                          one scale per channel
//   vpart  fp32 [B][HK][nvchunk][D]                 per-chunk channel abs-max of V (the V scales' first pass)
//   anchor int32 [B][HK]                            anchor key row or -1
//   arow   bf16 [B][HK][D]                          the anchor row as the keys are shifted by it (the key row as
//                                                   the prep sees it: raw, or normalised and rotated); zeros if none
//   part   fp32 [part_n][256][D] then [part_n][256][2]  the attention's split pieces (see AttnArgs): each piece's
//                                                   unnormalised rows (O times the V scales) and (reference, row sum)
// Scale granularity (per query row; per 16 keys; per channel) is this library's choice. The reference's per-thread
// groups follow its mma fragment layout (kernels/cuda/minimax/kitchen/quant_qk_int8.cu:245-247); the arithmetic
// inside a group is the reference's.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace lr {
namespace i8 {

constexpr int KGROUP = 16;    // keys per K scale
constexpr int VCHUNK = 256;   // keys per V abs-max partial
constexpr int AUX_BYTES = 1024;
constexpr int AUX_KS_OFF = 512;  // byte offset of the K scales in an aux block

// Tile width: 128 keys past 1024 keys at head dim 128, else 64 (launch.zig:333, kitchen_launch.cu:107).
inline int cta_for(int Sk, int D) { return D >= 128 && Sk > 1024 ? 128 : 64; }
// Hadamard of Q and K: H4 blocks up to 256 keys, else the signed H128 / plain H64 (kitchen_launch.cu:233-241,
// launch.zig:387-391).
inline int rotation_for(int Sk, int D) { return Sk <= 256 ? 4 : D; }

constexpr int SPLIT_MAX = 4;        // key ranges a split query block is cut into
constexpr int PART_PIECES = 256;    // pieces the partial area holds at most

struct Plan {
    int d, cta, ntiles, skp, nvchunk, rot, part_n;
    size_t q8, k8, vt, aux, qs, vs, vpart, anchor, arow, part, total;
};

inline size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

inline Plan plan_of(int B, int H, int HK, int Sq, int Sk, int D) {
    Plan p;
    p.d = D;
    p.cta = cta_for(Sk, D);
    p.ntiles = (Sk + p.cta - 1) / p.cta;
    p.skp = p.ntiles * p.cta;
    p.nvchunk = (Sk + VCHUNK - 1) / VCHUNK;
    p.rot = rotation_for(Sk, D);
    const size_t bh = (size_t)B * H, bhk = (size_t)B * HK;
    size_t at = 0;
    auto take = [&](size_t bytes) {
        const size_t o = at;
        at = align256(at + bytes);
        return o;
    };
    p.q8 = take(bh * Sq * D);
    p.k8 = take(bhk * p.skp * D);
    p.vt = take(bhk * p.skp * D);
    p.aux = take(bhk * p.ntiles * AUX_BYTES);
    p.qs = take(bh * Sq * 4);
    p.vs = take(bhk * D * 4);
    p.vpart = take(bhk * p.nvchunk * D * 4);
    p.anchor = take(bhk * 4);
    p.arow = take(bhk * D * 2);
    // the attention's split pieces: at most SPLIT_MAX a query block of 256 rows, PART_PIECES in all; none below
    // 4 SPLIT_MAX key tiles, where launch_attention never cuts
    const size_t nblk = bh * (size_t)((Sq + 255) / 256);
    p.part_n = p.ntiles < 4 * SPLIT_MAX ? 0
             : (int)(nblk * SPLIT_MAX < (size_t)PART_PIECES ? nblk * SPLIT_MAX : (size_t)PART_PIECES);
    p.part = take((size_t)p.part_n * 256 * (D + 2) * 4);
    p.total = at;
    return p;
}

// LDS / workspace swizzles (16-byte chunk index XOR). k_swz: the K operand read (lanes 0..15 take rows
// key_perm(0..15)) hits distinct chunk positions per 8 lanes and distinct (row parity, position) per 16 lanes; with
// 64-byte rows (head dim 64, four chunks a row, two rows a bank line) the lanes of each group of 8 take distinct
// (row parity, chunk) pairs. v_swz: the same property for V^T rows read 32 consecutive dims at a time.
__host__ __device__ inline int k_swz(int r, int D) {
    return D == 128 ? ((r >> 2) & 4) | ((((r >> 2) ^ r) & 1) << 1) | ((r >> 1) & 1)
                    : ((r >> 1) & 1) | (((r >> 4) & 1) << 1);
}
__host__ __device__ inline int v_swz(int d, int cta) {
    return cta == 128 ? (((d >> 1) & 7) ^ ((d & 1) << 2)) : (((d >> 1) ^ (d >> 3)) & 3);
}

struct PrepArgs {
    const uint16_t* q;  // bf16, element (b, h, n, c) at q + b*q_sb + h*q_sh + n*q_sn + c
    const uint16_t* k;
    const uint16_t* v;
    int64_t q_sb, q_sh, q_sn, k_sb, k_sh, k_sn, v_sb, v_sh, v_sn;
    int B, H, HK, Sq, Sk;
    uint8_t* ws;
    Plan p;
    // Kitchen.rmsRope fused into the prep (lr_int8_attention_prep_rope; rope_tab null: off). Every q and k row is
    // first normalised and rotated as the standalone pass stores it -- bf16 weights qw / kw [D], split-half pairs
    // (i, i + rope_rot / 2) from the bf16 table rope_tab [tokens][rope_rot / 2][2][2] (row stride tab_rs elements;
    // token n of any batch and head uses row n), the normalised value rounded to bf16 before the rotation -- and the
    // result is rounded to bf16 and quantised without being written back. Head dim 128, Sq == Sk.
    const uint16_t* rope_tab;
    int64_t tab_rs;
    const uint16_t* qw;
    const uint16_t* kw;
    int rope_rot;
    float rope_eps;
};

struct AttnArgs {
    uint8_t* ws;   // read, and (split blocks) written in its partial area
    uint16_t* out;  // bf16, element (b, h, n, c) at out + b*o_sb + h*o_sh + n*o_sn + c
    int64_t o_sb, o_sh, o_sn;
    int B, H, HK, G, Sq, Sk;
    float c;  // scale * log2(e)
    Plan p;
    // Query blocks (256 rows of one head) 0 .. nwhole - 1 run whole, one workgroup each; the rest (the last partial
    // round of the device's compute units) are cut into P key ranges each, one workgroup a range, whose rows go to the
    // partial area (part: the workspace's, Plan::part) and are merged by a second launch. Set by launch_attention.
    int nwhole, P;
    float* part;
};

hipError_t launch_prep(const PrepArgs& a, hipStream_t stream);
// cus: the device's compute units (the split of the last partial round of query blocks is chosen for them)
hipError_t launch_attention(AttnArgs a, int cus, hipStream_t stream);

}  // namespace i8
}  // namespace lr
