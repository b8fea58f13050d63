// Persistent streaming joint attention for gfx950: bf16 in, fp32 MFMA accumulation and softmax, bf16 out, over keys
// prepared as tile images (tile_image.h, written by kv_image.hip) or, in the key-rows instantiation, gathered into the
// same tile layout in LDS straight from the caller's key rows, and values read as they are, as bf16 rows.
//
// Semantics: the reference's kernels/cuda/qwen_image/attention.cu:253-444 (pattn2_kernel) as launched by
// src/engines/qwen_image/ops_launch.zig:163-172: O_i = softmax_j(scale <q_i, k_j>) v_j over keys j < nkeys (and
// j <= p0 + i when causal, attention.cu:304), query head h reading kv head h / (H / HK) (attention.cu:264-266), P
// rounded to bf16 for the P V product (attention.cu:418-424), output rounded to bf16 (attention.cu:432-443). The
// queries arrive normalised and rotated (bf16 rows, the reference's rope_q output, dit.zig:252-257), the keys as tile
// images or rows, the values as rows.
//
// Design (two waves per SIMD, 8 waves = 256 queries per block, 32 queries per wave; each 1 KB operand fragment read
// from LDS feeds one v_mfma_f32_32x32x16_bf16, 128 bytes per clock per CU at the MFMA rate, half of gfx950's LDS read
// bandwidth; the two waves of a SIMD overlap one's softmax VALU work and LDS reads with the other's MFMAs):
//
//  * Persistent: one workgroup per CU walks the blocks logical, logical + nwg, ... (a last partial pass shared by the
//    XCDs; or, split, cut into key ranges over all workgroups) and its key/value tiles form one
//    continuous stream through two 4-stage LDS rings (64 KB each). The loads of the next block's first tiles are in
//    flight while the current block finishes, and the query prologue of the next block follows the previous block's
//    epilogue without a kernel boundary.
//  * Key tile images: a key tile is stored in HBM as the LDS image of its 16 fragments, so each ring refill is two
//    contiguous 1 KB direct global->LDS loads per wave (one M0 write, immediate offsets), and each fragment read is one
//    conflict-free ds_read_b128 at an immediate offset from a per-step base: no per-fragment address arithmetic.
//  * Values as rows: a value tile (64 rows of 256 bytes at the caller's row stride) is brought into LDS by the same
//    direct loads, each lane fetching the 16-byte chunk that belongs at its LDS position in the "row-block" layout
//    (vt_offset below: 4-row x 64-byte blocks of 256 contiguous bytes); the P V operand (V^T, 8 consecutive keys of one
//    dim per lane) is then two ds_read_b64_tr_b16 (transposed) reads at immediate offsets from one per-lane base, with
//    no bank conflicts. The preparation launch no longer writes, and this kernel no longer reads, a value image.
//  * Step (one 64-key tile, 32 MFMA slots per wave): two half-steps of 16 slots; half-step j runs the 8 score MFMAs of
//    the next 32-key half-tile (S(j+1) = K Q^T, accumulator starting at -m) and the 8 P V MFMAs of the previous one
//    (O += V^T P(j-1)), while the VALU turns S(j) into P(j): one word (two keys of one query) per two slots, exp2 in
//    the even slot, bf16 pack and the fp32 row sum in the odd slot. Scores and P are double-buffered by half-tile.
//    Fragments are read three ahead into a register ring; one barrier per step, after a vmcnt wait that leaves the
//    step's own refills in flight.
//  * Softmax against a fixed reference: m = ceil of the exact maximum of the block's first 32 scores in the exp2
//    domain (c = scale * log2 e times the raw q.k product; the queries arrive normalised and rotated as the
//    reference's rope writes them, bf16), held as m / c and subtracted by the score MFMAs themselves, so
//    P = exp2(c S') with one multiply per score beside the exp. Softmax is shift-invariant: exact while P, the row
//    sums and O stay finite, i.e. unless a later key scores ~128 above m. The epilogue checks every row; a wave with a
//    non-finite row marks the block and, after the streaming loop, recomputes its 32 queries with the exact row
//    maximum (a two-pass form that reads key fragments and value rows straight from HBM and needs no LDS), so the
//    output never depends on the fixed reference.
#include "lr_common.h"
#include "lr_kernels.h"
#include "tile_image.h"

namespace lr {

namespace {

#include "attn_common.inc"

constexpr int SW = 8;             // waves per workgroup, two per SIMD
constexpr int SBM = 32 * SW;      // queries per block
constexpr int RING = 4;           // stages of each LDS ring
constexpr int RA = 3;             // fragments read ahead
constexpr int FR = 4;             // fragment ring entries
constexpr int WQ = IMG_TILE_BYTES / SW;   // bytes of a tile each wave loads
constexpr int MAX_WG_BLOCKS = 1024;      // whole blocks one workgroup may walk (launch_stream splits larger calls)
constexpr int REDO_WORDS = (MAX_WG_BLOCKS + 2 + 31) / 32;   // per wave: a bit per work item, for exact recomputation
constexpr int PMAX = 4;                   // pieces a cut block is split into at most
// one wave's partial of a cut block: its O^T registers (64 fp32 x 64 lanes, as 16 groups of 4 registers, 1 KB per
// group) and (m, l) per lane
constexpr int SLOT_WAVE_BYTES = 64 * 64 * 4 + 64 * 8;
static_assert(SW * SLOT_WAVE_BYTES == STREAM_SLOT_BYTES, "partial slot size");

// S = K Q^T with the accumulator starting at 0 / at c, and S += K Q^T: scores in VGPRs (the VALU reads them), Q in
// AGPRs. Inline asm, so the compiler cannot move the 64 Q registers into VGPRs; every VALU read of a result below is
// at least 16 MFMA slots after the MFMA, or behind a fence.
__device__ __forceinline__ void qk_zero(f32x16& d, const bf16x8& k, const bf16x8& q) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(k), "a"(q));
}
__device__ __forceinline__ void qk_init(f32x16& d, const bf16x8& k, const bf16x8& q, const f32x16& c) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %3" : "=&v"(d) : "v"(k), "a"(q), "v"(c));
}
__device__ __forceinline__ void qk_acc(f32x16& d, const bf16x8& k, const bf16x8& q) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(k), "a"(q));
}
// O += V^T P: the builtin, so that the compiler knows it is an MFMA (O stays in AGPRs, hazards are its job)
__device__ __forceinline__ void pv(f32x16& o, const bf16x8& v, const u32x4& p) {
    o = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v, __builtin_bit_cast(bf16x8, p), o, 0, 0, 0);
}
#define LR_NOP48 "s_nop 15\n\ts_nop 15\n\ts_nop 15"
__device__ __forceinline__ void fence_s(f32x16& s) { asm volatile(LR_NOP48 : "+v"(s)); }
__device__ __forceinline__ void fence_q8(bf16x8 (&q)[8]) {
    asm volatile(LR_NOP48 : "+a"(q[0]), "+a"(q[1]), "+a"(q[2]), "+a"(q[3]), "+a"(q[4]), "+a"(q[5]), "+a"(q[6]),
                 "+a"(q[7]));
}

// Two contiguous 1 KB direct loads, global -> LDS: lane l's 16 bytes of load i come from gaddr + 1024 i + 16 l and
// land at LDS byte lds + 1024 i + 16 l (the instruction offset applies to both addresses).
__device__ __forceinline__ void dma2k(uint64_t gaddr, uint32_t voff, uint32_t lds) {
    LR_ASM_M0_BEGIN
    asm volatile(
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, %1 offset:0\n\t"
        "global_load_lds_dwordx4 %0, %1 offset:1024" ::"v"(voff),
        "s"(gaddr), "s"(lds)
        : "memory", "m0");
    LR_ASM_M0_END
}

// Value tile rows in LDS: the 16 bytes of dims 8 c .. 8 c + 7 of tile row r (r < 64, c < 16) sit at byte
// vt_offset(r, c) of the 16 KB slot: 4-row x 4-chunk blocks of 256 contiguous bytes, block (r >> 2, c >> 2) at
// 256 (4 (r >> 2) + (c >> 2)), row r & 3 of it at + 64 (r & 3), chunk c & 3 at + 16 (c & 3). The address a lane reads
// for value fragment (16-key step kk, 32-dim block db) is then additive: a per-lane part (VT_LANE) plus
// 4096 kk + 256 db (+ 1024 for the fragment's second four keys), all immediates.
__host__ __device__ constexpr int vt_offset(int r, int c) {
    return 256 * (4 * (r >> 2) + (c >> 2)) + 64 * (r & 3) + 16 * (c & 3);
}
// Direct loads of a value tile: wave w's load i (i < 2) fills the slot's bytes 2048 w + 1024 i + 16 l (lane l), i.e.
// rows 8 w + 4 i + vt_lane_row(l), chunk vt_lane_chunk(l) of the tile.
__host__ __device__ constexpr int vt_lane_row(int l) { return (l >> 2) & 3; }
__host__ __device__ constexpr int vt_lane_chunk(int l) { return 4 * (l >> 4) + (l & 3); }
// The per-lane part of a transposed fragment read: lane l = 16 g + s reads (ds_read_b64_tr_b16: each group of 16
// lanes takes a 4-row x 16-dim block, lane s pointing at row s >> 2, dims 4 (s & 3) .. +3, and gets dim s of the four
// rows) keys 8 (l >> 5) + (s >> 2) of dims 16 (g & 1) + 4 (s & 3) .. of the fragment's 32-dim block.
__host__ __device__ constexpr int vt_lane(int l) {
    return 2048 * (l >> 5) + 64 * ((l >> 2) & 3) + 32 * ((l >> 4) & 1) + 8 * (l & 3);
}

// Two 1 KB direct loads of value rows, global -> LDS: lane l's 16 bytes of load 0 come from gaddr + voff0 and land at
// LDS byte lds + 16 l; those of load 1 from gaddr + voff1 + 1024 to lds + 1024 + 16 l (the instruction offset applies
// to both addresses; voff1 = voff0 + 4 rows - 1024 >= 0).
__device__ __forceinline__ void dma2v(uint64_t gaddr, uint32_t voff0, uint32_t voff1, uint32_t lds) {
    LR_ASM_M0_BEGIN
    asm volatile(
        "s_mov_b32 m0, %3\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, %2 offset:0\n\t"
        "global_load_lds_dwordx4 %1, %2 offset:1024" ::"v"(voff0),
        "v"(voff1), "s"(gaddr), "s"(lds)
        : "memory", "m0");
    LR_ASM_M0_END
}
// The same two loads with their own M0 each and no instruction offset (the last, clamped tile of a head, whose
// offsets may be smaller than 1024; and the key gathers of a call over key rows, whose lanes' offsets are rows apart).
__device__ __forceinline__ void dma2_apart(uint64_t gaddr, uint32_t voff0, uint32_t voff1, uint32_t lds) {
    LR_ASM_M0_BEGIN
    asm volatile(
        "s_mov_b32 m0, %3\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, %2 offset:0\n\t"
        "s_add_u32 m0, %3, 0x400\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2 offset:0" ::"v"(voff0),
        "v"(voff1), "s"(gaddr), "s"(lds)
        : "memory", "m0", "scc");
    LR_ASM_M0_END
}
// Key rows gathered into a tile image: lane l's 16 bytes of the two fragments a wave fills (at LDS byte lds + 16 l and
// lds + 1024 + 16 l) are 8 dims of the same key row, 16 dims (32 bytes) apart: load 0 from gaddr + koff, load 1 from
// gaddr + koff + 32 (its instruction offset 32 also adds to the LDS address, so M0 takes the other 992 bytes).
__device__ __forceinline__ void dma2k_rows(uint64_t gaddr, uint32_t koff, uint32_t lds) {
    LR_ASM_M0_BEGIN
    asm volatile(
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, %1 offset:0\n\t"
        "s_add_u32 m0, %2, 0x3e0\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, %1 offset:32" ::"v"(koff),
        "s"(gaddr), "s"(lds)
        : "memory", "m0", "scc");
    LR_ASM_M0_END
}

typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;
// One value fragment (the A operand V^T of O^T += V^T P^T: lane l = 32 hf + n gets keys 8 hf .. 8 hf + 7 of dim n of
// the 16-key x 32-dim block) from the row-block LDS layout: addr = slot + VT_LANE + 4096 kk + 256 db.
__device__ __forceinline__ bf16x8 vfrag_at(uint32_t addr) {
    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(uintptr_t)addr);
    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(uintptr_t)(addr + 1024));
    return __builtin_shufflevector(__builtin_bit_cast(bf16x4, lo), __builtin_bit_cast(bf16x4, hi), 0, 1, 2, 3, 4, 5, 6,
                                   7);
}

template <bool B>
struct BoolTag {
    static constexpr bool value = B;
};
template <int N>
struct IntTag {
    static constexpr int value = N;
};

typedef __attribute__((address_space(3))) const bf16x8 lds_frag;
__device__ __forceinline__ bf16x8 frag_at(uint32_t addr) { return *(lds_frag*)(uintptr_t)addr; }

// Recompute wave `wave`'s 32 queries of a block with the exact row maximum (the rare case of a non-finite row under the
// fixed reference): pass 1 takes the maximum of every score, pass 2 accumulates P = exp2(S - max) <= 1, the row sums and
// O, and the rows are written. The prepared queries are read from a.q (the block's rows, not yet overwritten), the key
// fragments straight from the tile images in HBM (a 1 KB fragment is one 16-byte load per lane) or, KR, from the key
// rows (lane 32 hf + n: 16 bytes of key 32 j + key_perm(n) for fragment ks, the tile image's content), and the value
// fragments from the value rows (eight 2-byte loads per lane): nothing here touches LDS or waits for the other waves.
// Called after the streaming loop, so that its registers do not add to the loop's.
template <bool KR>
__device__ __forceinline__ void redo_exact(const AttnArgs& a, int head, int hk, int row0, int tiles, int wave) {
    const int lane = threadIdx.x & 63, n = lane & 31, hf = lane >> 5;
    const int wrow0 = row0 + wave * 32, qrow = wrow0 + n;
    const int T = (a.nkeys + IMG_TILE_KEYS - 1) / IMG_TILE_KEYS;
    const uint64_t head_off = (uint64_t)hk * T * IMG_TILE_BYTES + (uint64_t)lane * 16;
    const uint8_t* kh = reinterpret_cast<const uint8_t*>(a.k) + head_off;
    const uint16_t* krows = a.k + (int64_t)hk * a.k_hs + 8 * hf;
    const uint16_t* vh = a.v + (int64_t)hk * a.v_hs + n;   // dim n of this lane's 32-dim blocks
    bf16x8 qf[8];
    const uint16_t* src = a.q + (int64_t)min(qrow, a.W - 1) * a.q_rs + head * D + 8 * hf;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qf[ks] = *reinterpret_cast<const bf16x8*>(src + 16 * ks);
    int lim0 = a.nkeys;
    if (a.causal) lim0 = min(lim0, a.p0 + qrow + 1);
    auto scores = [&](int j, const f32x16& c) {
        const uint8_t* kt = kh + (uint64_t)(j >> 1) * IMG_TILE_BYTES + (j & 1) * 8 * IMG_FRAG_BYTES;
        // KR: keys past nkeys read the last row (finite; masked below)
        const uint16_t* kr = krows + (int64_t)min(32 * j + img_key_perm(n), a.nkeys - 1) * a.k_rs;
        f32x16 sr = c;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const bf16x8 kf = KR ? *reinterpret_cast<const bf16x8*>(kr + 16 * ks)
                                 : *reinterpret_cast<const bf16x8*>(kt + ks * IMG_FRAG_BYTES);
            sr = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], sr, 0, 0, 0);
        }
        const int lim = lim0 - (32 * j + 8 * hf);
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (!(16 * (r >> 3) + (r & 7) < lim)) sr[r] = -INFINITY;
        return sr;
    };
    float mx = -INFINITY;
    for (int j = 0; j < 2 * tiles; ++j) {
        const f32x16 sr = scores(j, f32x16{});
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sr[r]);
    }
    const float m = wave_pair_max(mx);
    const f32x16 nm = f32x16{} - (m > -INFINITY ? m : 0.0f);
    const float c = a.c;
    f32x16 o[4] = {};
    float ls = 0.0f;
    for (int j = 0; j < 2 * tiles; ++j) {
        const f32x16 sr = scores(j, nm);
        // value fragment x of the half-tile (16-key step x >> 2, 32-dim block x & 3): keys 32 j + 16 (x >> 2) +
        // 8 hf .. +7 of dim 32 (x & 3) + n, eight 2-byte loads (rows past nkeys read the last row: their P is 0)
        auto vfrag = [&](int x) {
            uint16_t e[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int key = min(32 * j + 16 * (x >> 2) + 8 * hf + i, a.nkeys - 1);
                e[i] = vh[(int64_t)key * a.v_rs + 32 * (x & 3)];
            }
            u32x4 w;
#pragma unroll
            for (int i = 0; i < 4; ++i) w[i] = (uint32_t)e[2 * i] | ((uint32_t)e[2 * i + 1] << 16);
            return __builtin_bit_cast(bf16x8, w);
        };
        u32x4 pr[2];
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            const float e0 = __builtin_amdgcn_exp2f(sr[8 * (w >> 2) + 2 * (w & 3)] * c);
            const float e1 = __builtin_amdgcn_exp2f(sr[8 * (w >> 2) + 2 * (w & 3) + 1] * c);
            pr[w >> 2][w & 3] = pack_bf16x2(e0, e1);
            ls += e0 + e1;
        }
#pragma unroll
        for (int x = 0; x < 8; ++x)
            o[x & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vfrag(x), __builtin_bit_cast(bf16x8, pr[x >> 2]),
                                                            o[x & 3], 0, 0, 0);
    }
    const float inv = 1.0f / wave_pair_sum(ls);
    if (qrow < a.W) {
        uint16_t* dst = a.out + (int64_t)qrow * a.o_rs + head * D + 4 * hf;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int gg = 0; gg < 4; ++gg) {
                u32x2 w;
                w[0] = pack_bf16x2(o[db][4 * gg] * inv, o[db][4 * gg + 1] * inv);
                w[1] = pack_bf16x2(o[db][4 * gg + 2] * inv, o[db][4 * gg + 3] * inv);
                *reinterpret_cast<u32x2*>(dst + 32 * db + 8 * gg) = w;
            }
    }
}

// KR: a.k holds key rows (key j of kv head g at a.k + g * a.k_hs + j * a.k_rs), gathered into the tile-image layout by
// the ring's direct loads; otherwise a.k holds the tile images.
template <bool KR>
__global__ __launch_bounds__(SW * 64, 1) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_stream_kernel(AttnArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t Kr[RING * IMG_TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) uint8_t Vr[RING * IMG_TILE_BYTES];
    // per wave: bit n set = the wave's rows of the workgroup's n-th work item must be recomputed exactly
    __shared__ uint32_t redo_bits[SW][REDO_WORDS];
    __shared__ int arrival;   // a cut block's arrival count before this workgroup's piece, broadcast to the waves
    // this workgroup's tail pieces (at most two): head, row0, t0, t1, tail block, pieces of the block, index of this
    // piece, then the partial slot of every piece of the block
    __shared__ int tailtab[2][8 + PMAX];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 31, hf = lane >> 5;

    // XCD-aware order: hardware workgroup b runs on XCD b % 8; each XCD takes a contiguous range of logical ids, so
    // the blocks it runs at any time are consecutive query blocks of one or two heads (their K/V stay in its L2)
    const int nwg = gridDim.x, b = blockIdx.x;
    const int per = nwg >> 3, rem8 = nwg & 7, xcd = b & 7, idx = b >> 3;
    const int logical = xcd < rem8 ? xcd * (per + 1) + idx : rem8 * (per + 1) + (xcd - rem8) * per + idx;
    const int nqb = (a.W + SBM - 1) / SBM;
    const int nblk = nqb * a.H;
    const int T = (a.nkeys + IMG_TILE_KEYS - 1) / IMG_TILE_KEYS;
    // bytes from one kv head's keys to the next: its tile images, or (KR) the caller's kv-head stride
    const uint64_t head_bytes = KR ? (uint64_t)a.k_hs * 2 : (uint64_t)T * IMG_TILE_BYTES;

    // ---- the work of this workgroup. Whole blocks: logical, logical + nwg, ... for the nwhole / nwg full passes over
    // the workgroups; a last, partial pass of r = nwhole % nwg blocks (no split) is shared by the XCDs in proportion to
    // their workgroups (XCD x, holding logical ids f .. f + n - 1, takes the contiguous blocks from
    // base + r f / nwg to base + r (f + n) / nwg), so that no XCD idles while another runs two blocks a CU. With a.split, the
    // blocks from nwhole on (fewer than nwg, the "tail") are laid end to end as U = rem * T key tiles, and tail
    // workgroup L < a.tail_wg takes tiles [L U / tail_wg, (L + 1) U / tail_wg): at most two pieces, the end of one
    // block and the start of the next. A cut block's pieces each leave a partial (O, m, l); the last to arrive
    // merges them in piece order (deterministic) and writes the rows. A workgroup runs its tail pieces first and its
    // whole blocks after them, so that the merges overlap other workgroups' work instead of ending the kernel.
    const int nwhole = a.split ? (nblk / nwg) * nwg : nblk;
    const int nt = a.split ? a.tail_wg : 0;
    const int64_t U = (int64_t)(nblk - nwhole) * T;
    const int full = nwhole / nwg, r_last = nwhole - full * nwg;
    const int xf = logical - idx, xn = per + (xcd < rem8 ? 1 : 0);   // this XCD's first logical id and workgroups
    const int last0 = (int)((int64_t)r_last * xf / nwg);                // this XCD's first block of the last pass
    const int last_n = (int)((int64_t)r_last * (xf + xn) / nwg) - last0;
    const int n_whole = full + (idx < last_n ? 1 : 0);
    int64_t u0 = 0, u1 = 0;
    if (logical < nt) {
        u0 = (int64_t)logical * U / nt;
        u1 = (int64_t)(logical + 1) * U / nt;
    }
    const int n_pieces = u1 > u0 ? (int)((u1 - 1) / T - u0 / T + 1) : 0;
    const int nitems = n_whole + n_pieces;
    if (nitems == 0) return;
    if (tid < n_pieces) {
        // tail piece k = tid of this workgroup; tail workgroup owning tail tile u: ceil((u + 1) nt / U) - 1. 32-bit
        // arithmetic when every product fits (the usual case), else 64-bit.
        auto fill = [&](auto zero) {
            using I = decltype(zero);
            const I UU = (I)U, TT = (I)T, NT = (I)nt, uu0 = (I)u0, uu1 = (I)u1;
            auto owner = [&](I u) { return (int)(((u + 1) * NT + UU - 1) / UU) - 1; };
            const int k = tid;
            const I i = uu0 / TT + (I)k;
            const int blk = nwhole + (int)i;
            const int head = blk / nqb;
            const int lf = owner(i * TT), ll = owner((i + 1) * TT - 1);
            int* e = tailtab[k];
            e[0] = head;
            e[1] = (blk - head * nqb) * SBM;
            e[2] = k == 0 ? (int)(uu0 - i * TT) : 0;
            e[3] = (int)(uu1 - i * TT < TT ? uu1 - i * TT : TT);
            e[4] = (int)i;
            e[5] = ll - lf + 1;
            e[6] = logical - lf;
            for (int j = 0; j < PMAX; ++j) {
                const int wl = min(lf + j, ll);
                e[8 + j] = 2 * wl + (i == ((I)wl * UU / NT) / TT ? 0 : 1);
            }
        };
        if ((U + 1) * (int64_t)nt < ((int64_t)1 << 31)) fill(0u);
        else fill((uint64_t)0);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    block_barrier();

    struct Item {
        int head, hk, row0, t0, t1;
        int tail;   // tail piece (0 or 1) of this workgroup; -1 for a block computed whole
    };
    auto item_of = [&](int it) __attribute__((always_inline)) {
        Item r;
        if (it >= n_pieces) {
            const int pass = it - n_pieces;
            const int blk = pass < full ? logical + pass * nwg : full * nwg + last0 + idx;
            r.head = blk / nqb;
            r.row0 = (blk - r.head * nqb) * SBM;
            r.t0 = 0;
            r.t1 = T;
            r.tail = -1;
        } else {
            const int k = it;
            r.head = __builtin_amdgcn_readfirstlane(tailtab[k][0]);
            r.row0 = __builtin_amdgcn_readfirstlane(tailtab[k][1]);
            r.t0 = __builtin_amdgcn_readfirstlane(tailtab[k][2]);
            r.t1 = __builtin_amdgcn_readfirstlane(tailtab[k][3]);
            r.tail = k;
        }
        r.hk = r.head / a.G;
        if (a.causal) r.t1 = min(r.t1, (a.p0 + min(r.row0 + SBM, a.W) - 1) / IMG_TILE_KEYS + 1);
        return r;
    };

    // ---- the tile stream: cursors of the next key / value tile to load. Keys: this wave's WQ bytes of the tile image
    // (KR: row 0 of the tile in the kv head's key rows, each lane adding its own row and dims); values: row 0 of the
    // tile in the kv head's rows (each lane adds its own row and chunk offset).
    struct Cursor {
        int it, t, t1;
        uint64_t addr;
    };
    const uint64_t kimg = (uint64_t)(uintptr_t)a.k, vrows = (uint64_t)(uintptr_t)a.v;
    const uint32_t rowb = (uint32_t)a.v_rs * 2u;   // bytes per value row (< 2^25: launch_stream checks)
    const uint64_t vtile = (uint64_t)IMG_TILE_KEYS * rowb;
    // KR: bytes per tile of 64 key rows (< 2^31: launch_stream checks the row stride)
    const uint32_t ktile = KR ? (uint32_t)a.k_rs * (2u * IMG_TILE_KEYS) : (uint32_t)IMG_TILE_BYTES;
    auto k_at = [&](const Item& r) __attribute__((always_inline)) {
        if constexpr (KR) return kimg + (uint64_t)r.hk * head_bytes + (uint64_t)r.t0 * ktile;
        else return kimg + (uint64_t)r.hk * head_bytes + (uint64_t)r.t0 * IMG_TILE_BYTES + (uint64_t)wave * WQ;
    };
    auto v_at = [&](const Item& r) __attribute__((always_inline)) {
        return vrows + (uint64_t)r.hk * (uint64_t)a.v_hs * 2 + (uint64_t)r.t0 * vtile;
    };
    auto cur_start = [&](auto at) __attribute__((always_inline)) {
        const Item r = item_of(0);
        return Cursor{0, r.t0, r.t1, at(r)};
    };
    // past the last tile of the last item the cursor stays put: its loads refill a free ring slot with a tile that is
    // never read
    auto cur_next = [&](Cursor& c, auto step, auto at) __attribute__((always_inline)) {
        if (c.t + 1 < c.t1) {
            ++c.t;
            c.addr += step;
        } else if (c.it + 1 < nitems) {
            ++c.it;
            const Item r = item_of(c.it);
            c.t = r.t0;
            c.t1 = r.t1;
            c.addr = at(r);
        }
    };
    const uint32_t voff = (uint32_t)lane * 16u;
    const uint32_t kr0 = lds_addr(Kr), vr0 = lds_addr(Vr);
    // the value rows this lane loads: rows vrow and vrow + 4 of a tile, chunk vt_lane_chunk(lane)
    const uint32_t vrow = (uint32_t)(8 * wave + vt_lane_row(lane));
    const uint32_t vchunk = (uint32_t)(16 * vt_lane_chunk(lane));
    const uint32_t vo0 = vrow * rowb + vchunk, vo1 = vo0 + 4 * rowb - 1024;
    const int vfull = a.nkeys >> 6;   // value tiles t < vfull hold 64 rows; tile vfull (when nkeys % 64) fewer
    // KR: this wave fills fragments 2 wave and 2 wave + 1 of the image (32-key block mb = wave >> 2, k-steps
    // 2 (wave & 3) and + 1): lane 32 hf + n takes key row 32 mb + key_perm(n), dims 32 (wave & 3) + 8 hf .. +7, and
    // the 8 dims 16 further on (img_k_offset)
    // (computed at each load from the lane's byte offset, opaque to the compiler: nothing extra stays live in the loop)
    // ring slot x: byte offset x * 16 KB; this wave's loads fill its WQ bytes of the slot
    auto load_k = [&](Cursor& c, int pos) __attribute__((always_inline)) {
        const uint32_t lds = kr0 + (uint32_t)((pos & (RING - 1)) * IMG_TILE_BYTES) + (uint32_t)wave * WQ;
        if constexpr (KR) {
            uint32_t l16 = voff;   // 16 lane
            int w = wave;
            asm volatile("" : "+v"(l16), "+s"(w));
            const uint32_t krow = (uint32_t)(32 * (w >> 2)) + (uint32_t)img_key_perm((int)(l16 >> 4) & 31);
            const uint32_t kcol = (uint32_t)(64 * (w & 3)) + ((l16 >> 5) & 16u);
            // rows past nkeys (the head's last, partial tile) read the last row: finite, and their scores are masked
            const uint32_t lim = c.t < vfull ? 63u : (uint32_t)(a.nkeys - 1 - IMG_TILE_KEYS * c.t);
            dma2k_rows(c.addr, min(krow, lim) * (ktile / IMG_TILE_KEYS) + kcol, lds);
        } else {
            dma2k(c.addr, voff, lds);
        }
        cur_next(c, ktile, k_at);
    };
    auto load_v = [&](Cursor& c, int pos) __attribute__((always_inline)) {
        const uint32_t lds = vr0 + (uint32_t)((pos & (RING - 1)) * IMG_TILE_BYTES) + (uint32_t)wave * WQ;
        if constexpr (KR) {   // the lane's rows and chunk recomputed here, as for the keys (vrow, vchunk)
            uint32_t l16 = voff;
            int w = wave;
            asm volatile("" : "+v"(l16), "+s"(w));
            const uint32_t r = (uint32_t)(8 * w) + ((l16 >> 6) & 3u);
            const uint32_t ch = ((l16 >> 2) & 0xc0u) + (l16 & 0x30u);
            const uint32_t lim = c.t < vfull ? 63u : (uint32_t)(a.nkeys - 1 - IMG_TILE_KEYS * c.t);
            dma2_apart(c.addr, min(r, lim) * rowb + ch, min(r + 4, lim) * rowb + ch, lds);
        } else if (c.t < vfull) {
            dma2v(c.addr, vo0, vo1, lds);
        } else {   // the head's last, partial tile: rows past nkeys read the last row (finite; their P is 0)
            const uint32_t lim = (uint32_t)(a.nkeys - 1 - IMG_TILE_KEYS * c.t);
            dma2_apart(c.addr, min(vrow, lim) * rowb + vchunk, min(vrow + 4, lim) * rowb + vchunk, lds);
        }
        cur_next(c, vtile, v_at);
    };

    // ---- registers
    bf16x8 qa[8];      // AGPR-resident queries (B operand of S^T = K Q^T), per k-step
    f32x16 o[4];       // O^T accumulators, per 32-dim block
    f32x16 s[2];       // scores, per half-tile parity
    u32x4 p[2][2];     // P, [half-tile parity][16-key step of the half-tile]
    f32x16 negm;       // -m / c in every slot: the initial accumulator of the score MFMAs
    float mref = 0.0f; // m: the item's fixed softmax reference of this lane's query (exp2 domain)
    float ls = 0.0f;   // this lane's partial row sum (its 8 keys of every 16-key step)
    bf16x8 fr[FR];     // fragment ring
    const uint32_t lane16 = (uint32_t)lane * 16u;
    const uint32_t vlane = (uint32_t)vt_lane(lane);   // per-lane part of every value fragment read
    // the immediate part of value fragment x (16-key step x >> 2, 32-dim block x & 3) of a tile
    auto vfrag_off = [](int x) __attribute__((always_inline)) { return 4096 * (x >> 2) + 256 * (x & 3); };

    // mask the scores sb of half-tile j (keys 32 j ..) against nkeys and, causal, the query's position
    auto mask_half = [&](f32x16& sb, int j, int wrow0) __attribute__((always_inline)) {
        int lim = a.nkeys;
        if (a.causal) lim = min(lim, a.p0 + wrow0 + n + 1);
        lim -= 32 * j + 8 * hf;
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (!(16 * (r >> 3) + (r & 7) < lim)) sb[r] = -INFINITY;
    };
    // first half-tile that needs a mask for this wave
    auto mask_from = [&](int wrow0) __attribute__((always_inline)) {
        int jm = a.nkeys >> 5;
        if (a.causal) jm = min(jm, (a.p0 + wrow0 + 1) >> 5);
        return jm;
    };

    // one P word: E = the two exp2 of word w of the scores into e0/e1; C = bf16 pack into the P buffer, and the fp32
    // pair into the row sum (as the reference, attention.cu:403-407). Word w of a half-tile: 16-key step kk2 = w >> 2,
    // j = w & 3: score registers 8 kk2 + 2 j, +1 (keys 16 kk2 + 8 hf + 2 j, +1 of the half-tile).
    float e0 = 0.0f, e1 = 0.0f;
    const float c = a.c;   // scale * log2 e: scores are raw q.k products, the exponent is their exp2-domain value
    auto stage_e = [&](const f32x16& sb, int w) __attribute__((always_inline)) {
        e0 = __builtin_amdgcn_exp2f(sb[8 * (w >> 2) + 2 * (w & 3)] * c);
        e1 = __builtin_amdgcn_exp2f(sb[8 * (w >> 2) + 2 * (w & 3) + 1] * c);
        asm volatile("" ::"v"(e0), "v"(e1));   // computed in this slot, not sunk towards the next use
    };
    auto stage_c = [&](u32x4 (&pb)[2], int w) __attribute__((always_inline)) {
        const uint32_t x = pack_bf16x2(e0, e1);
        pb[w >> 2][w & 3] = x;
        const float es = e0 + e1;
        ls += es;
        asm volatile("" ::"v"(x), "v"(ls));
    };

    // ---- one half-step of 16 MFMA slots. QK: S so of the next half-tile from fragments 0-7 (k-steps); PV: O += the
    // V fragments 8-15 (16-key step (f - 8) >> 2, 32-dim block (f - 8) & 3) times P ppv; VALU: P po from S si.
    // rd(f) reads the fragment of position f (>= 16: the next half-step's position f - 16) into the ring.
    auto half_step = [&](f32x16& so, const u32x4 (&ppv)[2], const f32x16& si, u32x4 (&po)[2], auto qk_tag, auto pv_tag,
                         auto valu_tag, auto&& rd) __attribute__((always_inline)) {
        constexpr bool HAS_QK = decltype(qk_tag)::value;
        constexpr bool HAS_PV = decltype(pv_tag)::value;
        constexpr bool HAS_VALU = decltype(valu_tag)::value;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int f = 0; f < 16; ++f) {
            if (f < 8) {
                if constexpr (HAS_QK) {
                    if (f == 0) qk_init(so, fr[0], qa[0], negm);
                    else qk_acc(so, fr[f % FR], qa[f]);
                }
            } else {
                if constexpr (HAS_PV) pv(o[(f - 8) & 3], fr[f % FR], ppv[(f - 8) >> 2]);
            }
            if constexpr (HAS_VALU) {
                if ((f & 1) == 0) stage_e(si, f >> 1);
                else stage_c(po, f >> 1);
            }
            rd(f + RA);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    const BoolTag<true> yes{};
    const BoolTag<false> no{};

    // ---- per-item state
    int item = 0;
    Item cur = item_of(0);
    int g = 0;   // stream position of the current step (tile)

    // ---- the queries of item r (prepared rows: normalised and rotated as the reference's rope writes them, a.q with
    // row stride a.q_rs): this wave's 32 rows as the 8 B-operand fragments, loaded straight into the AGPRs. The loads
    // are asynchronous; LR_WAIT_Q(N) waits for them with N younger memory operations still in flight.
    auto load_q = [&](const Item& r) __attribute__((always_inline)) {
        const int qrow = min(r.row0 + wave * 32 + n, a.W - 1);
        const uint16_t* src = a.q + (int64_t)qrow * a.q_rs + r.head * D + 8 * hf;
        asm volatile(
            "global_load_dwordx4 %0, %8, off\n\t"
            "global_load_dwordx4 %1, %8, off offset:32\n\t"
            "global_load_dwordx4 %2, %8, off offset:64\n\t"
            "global_load_dwordx4 %3, %8, off offset:96\n\t"
            "global_load_dwordx4 %4, %8, off offset:128\n\t"
            "global_load_dwordx4 %5, %8, off offset:160\n\t"
            "global_load_dwordx4 %6, %8, off offset:192\n\t"
            "global_load_dwordx4 %7, %8, off offset:224"
            : "=a"(qa[0]), "=a"(qa[1]), "=a"(qa[2]), "=a"(qa[3]), "=a"(qa[4]), "=a"(qa[5]), "=a"(qa[6]), "=a"(qa[7])
            : "v"(src)
            : "memory");
    };
#define LR_WAIT_Q(N)                                                                                            \
    asm volatile("s_waitcnt vmcnt(" #N ")"                                                                      \
                 : "+a"(qa[0]), "+a"(qa[1]), "+a"(qa[2]), "+a"(qa[3]), "+a"(qa[4]), "+a"(qa[5]), "+a"(qa[6]),   \
                   "+a"(qa[7])::"memory")

    // ---- stream start: the first item's queries, K(0..2), V(0..1); the queries, K(0) and K(1) resident before
    // step 0
    Cursor kc = cur_start(k_at), vc = cur_start(v_at);
    for (int x = lane; x < REDO_WORDS; x += 64) redo_bits[wave][x] = 0u;
    load_q(cur);
    load_k(kc, 0);
    load_k(kc, 1);
    load_k(kc, 2);
    load_v(vc, 0);
    load_v(vc, 1);
    LR_WAIT_Q(6);
    block_barrier();

    // S(t0) of an item: the first half-tile's scores from key fragments 0-7 of slot kslot, accumulator at 0; then the
    // fixed reference m = ceil(max), S -= m / c, negm, O = 0, row sum 0
    auto first_scores = [&](const Item& r, uint32_t kslot) __attribute__((always_inline)) {
        const int wrow0 = r.row0 + wave * 32;
        uint32_t kb0 = kslot + lane16;
        asm volatile("" : "+v"(kb0));   // opaque: offsets stay immediates, nothing is precomputed across the loop
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const bf16x8 kf = frag_at(kb0 + (uint32_t)(ks * IMG_FRAG_BYTES));
            if (ks == 0) qk_zero(s[0], kf, qa[0]);
            else qk_acc(s[0], kf, qa[ks]);
        }
        fence_s(s[0]);
        if (2 * r.t0 >= mask_from(wrow0)) mask_half(s[0], 2 * r.t0, wrow0);
        float mx = s[0][0];
#pragma unroll
        for (int q = 1; q < 16; ++q) mx = fmaxf(mx, s[0][q]);
        mx = wave_pair_max(mx);
        // m in the exp2 domain, held as m / c in score units: the MFMAs then leave S - m / c, and P = exp2(c (S - m / c))
        // (an error of m / c's rounding shifts every exponent of the row alike, which the normalisation cancels)
        const float m = mx > -INFINITY ? ceilf(mx * c) : 0.0f;
        const float mc = m / c;
        mref = m;
        negm = f32x16{} - mc;
        s[0] -= mc;
        ls = 0.0f;
#pragma unroll
        for (int db = 0; db < 4; ++db) o[db] = f32x16{};
        asm volatile(LR_NOP48 : "+v"(negm));
    };

    // the output rows of item r from this wave's 16 packed words (32-dim block db = i >> 2, dims 8 (i & 3) + 4 hf ..
    // +3): 16 buffer stores, always issued (rows at or past W fall outside the buffer range and are dropped), so that
    // the number of memory operations after the next item's query loads is fixed
    auto store_rows = [&](const Item& r, const u32x2 (&w)[16]) __attribute__((always_inline)) {
        const int nrows = min(a.W - r.row0, SBM);
        const uint32_t nrec = (uint32_t)((int64_t)nrows * a.o_rs * 2 - (int64_t)r.head * D * 2);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            a.out + (int64_t)r.row0 * a.o_rs + r.head * D, 0, (int)nrec, 0x00020000);
        uint32_t vo = (uint32_t)((wave * 32 + n) * a.o_rs * 2 + 8 * hf);
        asm volatile("" : "+v"(vo));   // computed here, the store offsets stay immediates
#pragma unroll
        for (int i = 0; i < 16; ++i)
            __builtin_amdgcn_raw_buffer_store_b64(w[i], rs, (int)(vo + 2 * (32 * (i >> 2) + 8 * (i & 3))), 0, 0);
    };
    // O / l of this wave's rows as packed bf16 words; returns true when a row is not finite (l >= 1/2 for every row,
    // the first half-tile's maximum has P >= 1/2, so only overflow makes one)
    auto pack_rows = [&](u32x2 (&w)[16], float l) __attribute__((always_inline)) {
        const float inv = 1.0f / l;
        float nan0 = 0.0f * l, nan1 = 0.0f, nan2 = 0.0f, nan3 = 0.0f;   // NaN iff some value is not finite
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int gg = 0; gg < 4; ++gg) {
                const float y0 = o[db][4 * gg] * inv, y1 = o[db][4 * gg + 1] * inv;
                const float y2 = o[db][4 * gg + 2] * inv, y3 = o[db][4 * gg + 3] * inv;
                nan0 = fmaf(y0, 0.0f, nan0);
                nan1 = fmaf(y1, 0.0f, nan1);
                nan2 = fmaf(y2, 0.0f, nan2);
                nan3 = fmaf(y3, 0.0f, nan3);
                w[4 * db + gg][0] = pack_bf16x2(y0, y1);
                w[4 * db + gg][1] = pack_bf16x2(y2, y3);
            }
        return (nan0 + nan1 + nan2 + nan3) != 0.0f;
    };
    // rows of item r (O / l) out; a wave with a non-finite row stores nothing and marks item it: after the streaming
    // loop it recomputes those rows exactly (its rows still hold the prepared queries when they are the output rows)
    auto write_rows = [&](const Item& r, int it, float l) __attribute__((always_inline)) {
        const int wrow0 = r.row0 + wave * 32;
        u32x2 w[16];
        const bool bad = pack_rows(w, l) && wrow0 + n < a.W;
        if (__builtin_amdgcn_ballot_w64(bad)) {
            if (lane == 0) redo_bits[wave][it >> 5] |= 1u << (it & 31);
        } else {
            store_rows(r, w);
        }
    };

    // a piece of a cut block: its partial out (sc1: coherent at device scope, not kept in this XCD's L2), then the
    // block's arrival count; the last piece to arrive reads the others' partials and writes the rows
    auto finish_piece = [&](const Item& r, int it) __attribute__((always_inline)) {
        const int* e = tailtab[r.tail];
        const int i = __builtin_amdgcn_readfirstlane(e[4]);
        const int np = __builtin_amdgcn_readfirstlane(e[5]);
        const float l = wave_pair_sum(ls);
        if (np == 1) {   // the whole block in one piece
            write_rows(r, it, l);
            return;
        }
        auto slot_rsrc = [&](int slot) __attribute__((always_inline)) {
            uint8_t* base = static_cast<uint8_t*>(a.part) + (int64_t)slot * STREAM_SLOT_BYTES + wave * SLOT_WAVE_BYTES;
            return __builtin_amdgcn_make_buffer_rsrc(base, 0, SLOT_WAVE_BYTES, 0x00020000);
        };
        {
            const __amdgpu_buffer_rsrc_t rs = slot_rsrc(__builtin_amdgcn_readfirstlane(e[8 + e[6]]));
#pragma unroll
            for (int gi = 0; gi < 16; ++gi) {
                f32x4 x;
#pragma unroll
                for (int e = 0; e < 4; ++e) x[e] = o[gi >> 2][4 * (gi & 3) + e];
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), rs, (gi * 64 + lane) * 16, 0, 16);
            }
            u32x2 ml;
            ml[0] = __float_as_uint(mref);
            ml[1] = __float_as_uint(l);
            __builtin_amdgcn_raw_buffer_store_b64(ml, rs, 64 * 64 * 4 + lane * 8, 0, 16);
        }
        LR_WAIT_VMCNT(0);
        block_barrier();   // every wave's partial is complete before the arrival is counted
        if (tid == 0) {
            arrival = __hip_atomic_fetch_add(a.cnt + i, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
        block_barrier();
        if (__builtin_amdgcn_readfirstlane(arrival) != np - 1) return;
        if (tid == 0) __hip_atomic_store(a.cnt + i, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // merge, in piece order: the weights 2^(m_j - M), then O and l as their weighted sums
        const int mine = __builtin_amdgcn_readfirstlane(e[6]);
        int slot_of[PMAX];
        float mj[PMAX], lj[PMAX];
        float mmax = -INFINITY;
#pragma unroll
        for (int j = 0; j < PMAX; ++j) {
            slot_of[j] = __builtin_amdgcn_readfirstlane(e[8 + j]);
            mj[j] = -INFINITY;
            lj[j] = 0.0f;
            if (j < np) {
                if (j == mine) {
                    mj[j] = mref;
                    lj[j] = l;
                } else {
                    const u32x2 ml = __builtin_amdgcn_raw_buffer_load_b64(slot_rsrc(slot_of[j]), 64 * 64 * 4 + lane * 8,
                                                                          0, 16);
                    mj[j] = __uint_as_float(ml[0]);
                    lj[j] = __uint_as_float(ml[1]);
                }
                mmax = fmaxf(mmax, mj[j]);
            }
        }
        float lsum = 0.0f;
#pragma unroll
        for (int j = 0; j < PMAX; ++j) {
            mj[j] = j < np ? __builtin_amdgcn_exp2f(mj[j] - mmax) : 0.0f;
            lsum += mj[j] * lj[j];
        }
        f32x4 acc[16];
#pragma unroll
        for (int gi = 0; gi < 16; ++gi) acc[gi] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < PMAX; ++j) {
            if (j < np) {
                f32x4 x[16];
                if (j == mine) {
#pragma unroll
                    for (int gi = 0; gi < 16; ++gi)
#pragma unroll
                        for (int e2 = 0; e2 < 4; ++e2) x[gi][e2] = o[gi >> 2][4 * (gi & 3) + e2];
                } else {   // one batch of 16 loads, then the products
                    const __amdgpu_buffer_rsrc_t rs = slot_rsrc(slot_of[j]);
#pragma unroll
                    for (int gi = 0; gi < 16; ++gi)
                        x[gi] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (gi * 64 + lane) * 16,
                                                                                                0, 16));
                }
#pragma unroll
                for (int gi = 0; gi < 16; ++gi) acc[gi] += mj[j] * x[gi];
            }
        }
#pragma unroll
        for (int gi = 0; gi < 16; ++gi)
#pragma unroll
            for (int e2 = 0; e2 < 4; ++e2) o[gi >> 2][4 * (gi & 3) + e2] = acc[gi][e2];
        LR_WAIT_VMCNT(0);
        write_rows(r, it, lsum);
    };

    // The end of an item (in the boundary step, V(g - 1) its last value tile): P of its last half-tile (S buffer 1)
    // into P buffer 1 beside the P V products of the half-tile before (P buffer 0, value fragments 0-7), then the
    // last P V products (P buffer 1, fragments 8-15), then its rows (or its partial).
    auto finish_item = [&](const Item& r, int it, uint32_t vslot) __attribute__((always_inline)) {
        const int wrow0 = r.row0 + wave * 32;
        if (2 * r.t1 - 1 >= mask_from(wrow0)) mask_half(s[1], 2 * r.t1 - 1, wrow0);
        uint32_t vb0 = vslot + vlane;
        asm volatile("" : "+v"(vb0));
        bf16x8 vf[4];
#pragma unroll
        for (int x = 0; x < 3; ++x) vf[x] = vfrag_at(vb0 + (uint32_t)vfrag_off(x));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int x = 0; x < 16; ++x) {
            if (x + 3 < 16) vf[(x + 3) & 3] = vfrag_at(vb0 + (uint32_t)vfrag_off(x + 3));
            pv(o[x & 3], vf[x & 3], (x < 8 ? p[0] : p[1])[(x >> 2) & 1]);
            if (x < 8) {
                stage_e(s[1], x);
                stage_c(p[1], x);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (r.tail < 0) write_rows(r, it, wave_pair_sum(ls));
        else finish_piece(r, it);
    };

    // a steady-state step over key tile g (both halves) and value tile g - 1. Fragment positions of the B half: 0-7
    // keys mb 0, 8-15 values mb 0, 16+ the A half's keys (mb 1); of the A half: 0-7 keys mb 1, 8-15 values mb 1, 16+
    // the next step's keys (mb 0).
    auto step = [&](const Item& r, int t) __attribute__((always_inline)) {
        const int wrow0 = r.row0 + wave * 32;
        const int jm = mask_from(wrow0);
        // per-step fragment bases (opaque to the compiler, so that every fragment offset below stays an immediate)
        uint32_t kb = kr0 + (uint32_t)((g & (RING - 1)) * IMG_TILE_BYTES) + lane16;
        uint32_t vb = vr0 + (uint32_t)(((g - 1) & (RING - 1)) * IMG_TILE_BYTES) + vlane;
        uint32_t kn = kr0 + (uint32_t)(((g + 1) & (RING - 1)) * IMG_TILE_BYTES) + lane16;
        asm volatile("" : "+v"(kb), "+v"(vb), "+v"(kn));
        auto rd_b = [&](int f) __attribute__((always_inline)) {
            if (f < 8) fr[f % FR] = frag_at(kb + f * IMG_FRAG_BYTES);
            else if (f < 16) fr[f % FR] = vfrag_at(vb + vfrag_off(f - 8));
            else fr[f % FR] = frag_at(kb + (f - 8) * IMG_FRAG_BYTES);
        };
        auto rd_a = [&](int f) __attribute__((always_inline)) {
            if (f < 8) fr[f % FR] = frag_at(kb + (8 + f) * IMG_FRAG_BYTES);
            else if (f < 16) fr[f % FR] = vfrag_at(vb + vfrag_off(f));
            else fr[f % FR] = frag_at(kn + (f - 16) * IMG_FRAG_BYTES);
        };
        // B half: j = 2t - 1
        if (2 * t - 1 >= jm) mask_half(s[1], 2 * t - 1, wrow0);
        load_k(kc, g + 3);
        half_step(s[0], p[0], s[1], p[1], yes, yes, yes, rd_b);
        // A half: j = 2t
        if (2 * t >= jm) mask_half(s[0], 2 * t, wrow0);
        load_v(vc, g + 2);
        half_step(s[1], p[1], s[0], p[0], yes, yes, yes, rd_a);
        LR_WAIT_VMCNT(6);   // K(g + 2) and V(g) have landed; only this step's refills and V(g + 1) may be in flight
        block_barrier();
    };

    // ---- the items of this workgroup
    Item prev = cur;
    bool has_prev = false;
    for (;;) {
        // boundary step g: the end of the previous item (value tile g - 1), the start of this one (key tile g)
        const uint32_t kslot = kr0 + (uint32_t)((g & (RING - 1)) * IMG_TILE_BYTES);
        if (has_prev) {
            load_q(cur);   // prev's queries are dead: its last score MFMA ran in the step before
            finish_item(prev, item - 1, vr0 + (uint32_t)(((g - 1) & (RING - 1)) * IMG_TILE_BYTES));
            LR_WAIT_Q(16);   // the 16 output stores of prev may still be in flight
        }
        first_scores(cur, kslot);
        load_k(kc, g + 3);
        load_v(vc, g + 2);
        // the A half of the item's first step: S(2 t0 + 1) from key fragments 8-15 into S buffer 1, P(2 t0) from S
        // buffer 0 into P buffer 0
        {
            uint32_t kb = kslot + lane16;
            uint32_t kn = kr0 + (uint32_t)(((g + 1) & (RING - 1)) * IMG_TILE_BYTES) + lane16;
            asm volatile("" : "+v"(kb), "+v"(kn));
            auto rd0 = [&](int f) __attribute__((always_inline)) {
                if (f < 8) fr[f % FR] = frag_at(kb + (8 + f) * IMG_FRAG_BYTES);
                else if (f >= 16) fr[f % FR] = frag_at(kn + (f - 16) * IMG_FRAG_BYTES);
            };
#pragma unroll
            for (int f = 0; f < RA; ++f) rd0(f);
            half_step(s[1], p[1], s[0], p[0], yes, no, yes, rd0);
        }
        LR_WAIT_VMCNT(6);
        block_barrier();
        ++g;
        for (int t = cur.t0 + 1; t < cur.t1; ++t) {
            step(cur, t);
            ++g;
        }
        prev = cur;
        has_prev = true;
        if (++item >= nitems) break;
        cur = item_of(item);
    }
    finish_item(prev, item - 1, vr0 + (uint32_t)(((g - 1) & (RING - 1)) * IMG_TILE_BYTES));
    LR_WAIT_VMCNT(0);   // no direct load is still writing LDS when the workgroup ends

    // ---- the rare exact recomputation of the marked items (a cut block: all of it, by the workgroup that merged it)
    for (int wd = 0; wd < (nitems + 31) / 32; ++wd) {
        uint32_t bits = __builtin_amdgcn_readfirstlane(redo_bits[wave][wd]);
        while (bits) {
            const int it = 32 * wd + __builtin_ctz(bits);
            bits &= bits - 1;
            Item r = item_of(it);
            if (a.causal) r.t1 = min(T, (a.p0 + min(r.row0 + SBM, a.W) - 1) / IMG_TILE_KEYS + 1);
            else r.t1 = T;
            redo_exact<KR>(a, r.head, r.hk, r.row0, r.t1, wave);
        }
    }
}

// the split tail's arrival counters, cleared (a fill kernel, not a memset: safe under graph capture)
__global__ __launch_bounds__(STREAM_MAX_WG) void zero_cnt_kernel(int* cnt) { cnt[threadIdx.x] = 0; }

}  // namespace

bool stream_split_params(int W, int H, int nkeys, int causal, int nwg, int* tail_wg) {
    const int64_t nblk = (int64_t)((W + SBM - 1) / SBM) * H;
    const int64_t rem = nblk % nwg;
    const int64_t T = (nkeys + IMG_TILE_KEYS - 1) / IMG_TILE_KEYS;
    // cut the tail when balancing it saves at least 4 key tiles per workgroup (a piece costs about a tile's time in
    // partial traffic and its boundary step)
    if (causal || rem == 0 || T * (nwg - rem) < 4 * (int64_t)nwg) return false;
    *tail_wg = (int)std::min<int64_t>(std::min<int64_t>(nwg, rem * T), rem * (PMAX - 1));
    return true;
}

hipError_t launch_stream(const AttnArgs& a, int nwg, hipStream_t stream, bool key_rows) {
    if (a.W < 1 || a.H < 1 || nwg < 1 || nwg > STREAM_MAX_WG) return hipErrorInvalidValue;
    // value (and key) rows: a lane's 32-bit load offset reaches 63 rows into a tile (< 2^31 bytes)
    if (a.v_rs < D || a.v_rs > STREAM_MAX_V_RS || a.v_rs % 8 || a.v_hs < 0 || a.v_hs % 8) return hipErrorInvalidValue;
    if (key_rows && (a.k_rs < D || a.k_rs > STREAM_MAX_V_RS || a.k_rs % 8 || a.k_hs < 0 || a.k_hs % 8))
        return hipErrorInvalidValue;
    // at most MAX_WG_BLOCKS whole blocks per workgroup (its recomputation bits): larger calls run as several launches
    // over consecutive query-row ranges (queries, outputs and, causal, the diagonal offset p0 shifted)
    const int64_t rows_per = (int64_t)SBM * std::max<int64_t>(1, (int64_t)MAX_WG_BLOCKS * nwg / a.H);
    bool cleared = false;
    for (int64_t r0 = 0; r0 < a.W; r0 += rows_per) {
        AttnArgs b = a;
        b.W = (int)std::min<int64_t>(rows_per, a.W - r0);
        b.q = a.q + r0 * a.q_rs;
        b.out = a.out + r0 * a.o_rs;
        b.p0 = a.p0 + (int)r0;
        const int64_t blocks = (int64_t)((b.W + SBM - 1) / SBM) * b.H;
        if (blocks > (int64_t)MAX_WG_BLOCKS * nwg) return hipErrorInvalidValue;
        b.split = 0;
        b.tail_wg = 0;
        int tw = 0;
        if (a.part && a.cnt && stream_split_params(b.W, b.H, b.nkeys, b.causal, nwg, &tw)) {
            b.split = 1;
            b.tail_wg = tw;
            // over key rows no preparation launch has cleared the arrival counters: a fill launch first (every launch
            // leaves them zero again)
            if (key_rows && !cleared) {
                hipLaunchKernelGGL(zero_cnt_kernel, dim3(1), dim3(STREAM_MAX_WG), 0, stream, a.cnt);
                const hipError_t e = hipGetLastError();
                if (e != hipSuccess) return e;
                cleared = true;
            }
        }
        const unsigned grid = b.split ? (unsigned)nwg : (unsigned)std::min<int64_t>(blocks, nwg);
        if (key_rows) hipLaunchKernelGGL(attn_stream_kernel<true>, dim3(grid), dim3(SW * 64), 0, stream, b);
        else hipLaunchKernelGGL(attn_stream_kernel<false>, dim3(grid), dim3(SW * 64), 0, stream, b);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace lr
