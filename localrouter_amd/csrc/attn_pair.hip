// Flash-style joint attention for gfx950 with 64 queries per wave ("pair" kernel): bf16 in, fp32 MFMA accumulation
// and softmax, bf16 out. Same semantics as the pipelined kernel in attn_fwd.hip, which follow the reference's
// kernels/cuda/qwen_image/attention.cu:253-444 (pattn2_kernel) as launched by
// src/engines/qwen_image/ops_launch.zig:163-172: O_i = softmax_j(scale <q_i, k_j>) v_j over keys j < nkeys (and
// j <= p0 + i when causal, attention.cu:304), query head h reading kv head h / (H / HK) (attention.cu:264-266), P
// rounded to bf16 for the PV product (attention.cu:418-424), output rounded to bf16 (attention.cu:432-443).
//
// Why 64 queries per wave. Every 32x32x16 MFMA takes one 1 KB operand fragment (a K or V^T slice) from LDS. On
// gfx950 one ds_read_b128 per MFMA holds the matrix pipe at about two thirds of its rate (LDS bandwidth), one per two
// MFMAs does not. A wave that owns two 32-query blocks feeds each fragment to two MFMAs. Its state does not fit the
// 256 VGPRs of two waves per SIMD, so the kernel runs one wave per SIMD (4 waves, 256 queries per workgroup) and
// places it explicitly: O (128) and Q (64) in AGPRs, which MFMAs read and write directly; scores, P and the fragment
// ring in VGPRs. The MFMAs are inline asm so that the compiler cannot move accumulators between the two files; the
// compiler does not see them as MFMAs, so every VALU read of an MFMA result below is either many MFMA slots after
// that MFMA or behind a fence_* (wait states that the registers they protect depend on).
//
// Per 64-key tile t a wave runs one step of 64 MFMA slots (one wave instruction stream, a sched_barrier per slot):
//   slots  0-23   O += V(t-1)^T P(t-1), fragments V0-V11   | VALU: P(t) of key block 0, words 11-15
//   slots 24-39   S(t+1) key block 0 = K(t+1) Q^T           | VALU: P(t) of key block 1, words 0-15
//   slots 40-47   O += V(t-1)^T P(t-1), fragments V12-V15   | VALU: P(t+1) of key block 0 from slot 42 on
//   slots 48-63   S(t+1) key block 1                        | VALU: P(t+1) of key block 0, words 0-10
// One P word (two keys of one query) every two slots, in three stages one slot apart (exp2; bf16 pack and pair sum;
// row sum), so that no VALU instruction waits on the one before it and the MFMA issue never waits on the VALU.
// Scores are single-buffered: a key block's exps finish before the MFMAs that overwrite it start. P is double-buffered
// (P(t) is written while P(t-1) is consumed). K and V^T tiles stream through a 4-stage LDS ring by direct
// global->LDS loads; the first three fragments of the next step are read before the step-closing barrier.
//
// Softmax reference. Each query's reference m is the ceil of its exact maximum over the first key tile (exp2 domain)
// and stays fixed: P = exp2(s - m), folded into the score MFMAs (their accumulator starts at -m), with no running max,
// no rescaling and no per-score VALU op. Softmax is shift-invariant, so this is exact as long as every P, the row sums
// and O stay finite; P can exceed 1 by up to 2^127 before that fails, i.e. only when a later key scores ~128 (exp2
// domain) above the first tile's maximum. The epilogue checks l and O of every row; a wave with a row that is not
// finite marks its first row with a NaN, and a second launch (the running-max kernel of attn_fwd.hip, over the same
// 256-query blocks) recomputes exactly the marked blocks.
//
// Stream-K (SK). 256-query blocks over a whole number of CUs leave the last round of workgroups part-empty (432 blocks
// on 256 CUs: 1.69 rounds of work in 2 rounds of time). The SK launch runs one workgroup per CU over the blocks' key
// tiles laid end to end (block-major) and gives workgroup c the tiles [c T / n, (c + 1) T / n). With at least as many
// blocks as workgroups a range holds the tail of one block, whole blocks, then the head of another, so a block is cut
// at most once, at the start c T / n of some range c. Both parts of a cut block store their unnormalised O, reference
// and per-lane row sums (the head part to slot 2c, the tail part to slot 2c + 1 of the partials area) and write no
// output; no workgroup waits for another. A second kernel (attn_sk_combine_kernel) merges each cut block's two parts,
// O = O1 2^(m1 - m) + O2 2^(m2 - m), l likewise, m = max, and writes its rows, marking overflow as the epilogue does.
#include "lr_common.h"
#include "lr_kernels.h"

namespace lr {

namespace {

#include "attn_common.inc"

// One 16-byte-per-lane ring load, buffer -> LDS: lane l reads 16 bytes at descriptor base + voff (zeros past the
// descriptor's record count) and they land at LDS byte address lds + 16 l. The descriptor and lds are wave-uniform.
__device__ __forceinline__ void dma16_buf(u32x4 rsrc, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc),
                 "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory");
}

// S = K Q^T (accumulator starts at 0, or at c); S += K Q^T, as inline asm: scores in VGPRs (the VALU reads them), Q in
// AGPRs.
__device__ __forceinline__ void mfma_qk0(f32x16& d, const bf16x8& k, const bf16x8& q) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(k), "a"(q));
}
__device__ __forceinline__ void mfma_qk_c(f32x16& d, const bf16x8& k, const bf16x8& q, const f32x16& c) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %3" : "=&v"(d) : "v"(k), "a"(q), "v"(c));
}
__device__ __forceinline__ void mfma_qk(f32x16& d, const bf16x8& k, const bf16x8& q) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(k), "a"(q));
}
// O += V^T P through the builtin: the compiler knows this one is an MFMA, so any copy it makes of O (which lives in
// AGPRs, the accumulator form it selects for a one-wave-per-SIMD kernel) gets the hazard waits it needs.
__device__ __forceinline__ void mfma_pv(f32x16& o, const bf16x8& v, const bf16x8& p) {
    o = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v, p, o, 0, 0, 0);
}
// Hazard fences: 48 wait states, more than any MFMA -> VALU or VALU -> MFMA dependency needs on gfx950. Each takes the
// registers it protects as in/out operands, so that no access to them can be scheduled across it.
#define LR_NOP48 "s_nop 15\n\ts_nop 15\n\ts_nop 15"
__device__ __forceinline__ void fence_o(f32x16 (&o)[2][4]) {
    asm volatile(LR_NOP48 : "+a"(o[0][0]), "+a"(o[0][1]), "+a"(o[0][2]), "+a"(o[0][3]), "+a"(o[1][0]), "+a"(o[1][1]),
                 "+a"(o[1][2]), "+a"(o[1][3]));
}
__device__ __forceinline__ void fence_s(f32x16 (&s)[2][2]) {
    asm volatile(LR_NOP48 : "+v"(s[0][0]), "+v"(s[0][1]), "+v"(s[1][0]), "+v"(s[1][1]));
}
__device__ __forceinline__ void fence_negm(f32x16 (&m)[2]) { asm volatile(LR_NOP48 : "+v"(m[0]), "+v"(m[1])); }
__device__ __forceinline__ void fence_q(bf16x8 (&q)[8]) {
    asm volatile(LR_NOP48 : "+a"(q[0]), "+a"(q[1]), "+a"(q[2]), "+a"(q[3]), "+a"(q[4]), "+a"(q[5]), "+a"(q[6]),
                 "+a"(q[7]));
}

template <bool B>
struct BoolTag {
    static constexpr bool value = B;
};

constexpr int PW = 4;                 // waves per workgroup
constexpr int PBM = 64 * PW;          // queries per workgroup
constexpr int PNS = 4;                // ring stages
constexpr int PTILE = BN * D;         // elements per K or V^T tile
constexpr int PLOADS = BN / 4 / PW;   // 1 KB direct loads per wave per tile

// stream-K partials: per slot and wave, O as [2 nb][4 db][4 gg][64 lanes] float4, then m and the per-lane row sums as
// [2 nb][2][64 lanes]
constexpr int SK_WAVE_FLOATS = 2 * 4 * 16 * 64 + 2 * 2 * 64;
constexpr int SK_ML = 2 * 4 * 16 * 64;   // offset of m, l in a wave's partial
static_assert(PW * SK_WAVE_FLOATS == SK_SLOT_FLOATS, "partial slot size");

// Cut point of stream-K range c (block, first tile of the tail part); tile 0 when the range starts at a block boundary
struct SkCut {
    int blk, t;
};
__device__ __forceinline__ SkCut sk_cut(int c, int nblk, int blk_tiles, int nwg) {
    const int64_t pos = (int64_t)c * ((int64_t)nblk * blk_tiles) / nwg;
    const int blk = (int)(pos / blk_tiles);
    return SkCut{blk, (int)(pos - (int64_t)blk * blk_tiles)};
}

template <int QK, bool VT, bool SK>
__global__ __launch_bounds__(PW * 64, 1) __attribute__((amdgpu_waves_per_eu(1, 1))) void attn_pair_kernel(AttnArgs a0) {
    // FOLD: fused queries arrive multiplied by scale * log2(e), so a score is already in the exp2 domain, and the
    // reference m is subtracted by the score MFMAs themselves (their accumulator starts at -m): P = exp2(S) with no
    // per-score VALU op. Plain queries keep exact raw scores: P = exp2(S * c - m).
    constexpr bool FOLD = QK != QK_PLAIN;
    typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;
    __shared__ __attribute__((aligned(1024))) uint16_t Kr[PNS * PTILE];
    __shared__ __attribute__((aligned(1024))) uint16_t Vr[PNS * PTILE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: LDS destinations stay in SGPRs
    const int n = lane & 31, hf = lane >> 5;

    // XCD-aware mapping: hardware workgroup b runs on XCD b % 8; each XCD gets a contiguous range of logical ids
    const int nwg = gridDim.x, b = blockIdx.x;
    const int per = nwg >> 3, rem = nwg & 7, xcd = b & 7, idx = b >> 3;
    const int logical = xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
    const int nqb = (a0.W + PBM - 1) / PBM;
    // SK: this workgroup's range of block-major key tiles; otherwise one whole block
    const int blk_tiles = (a0.nkeys + BN - 1) / BN;
    int64_t seg_pos = 0, seg_end = 1;
    if constexpr (SK) {
        const int64_t total = (int64_t)nqb * a0.H * blk_tiles;
        seg_pos = (int64_t)logical * total / nwg;
        seg_end = (int64_t)(logical + 1) * total / nwg;
    }
    const AttnArgs& a = a0;
    for (bool first_seg = true; seg_pos < seg_end; first_seg = false) {
    int blk = logical, t0 = 0, t1 = blk_tiles;
    if constexpr (SK) {
        blk = (int)(seg_pos / blk_tiles);
        t0 = (int)(seg_pos - (int64_t)blk * blk_tiles);
        t1 = (int)min((int64_t)blk_tiles, seg_end - (int64_t)blk * blk_tiles);
        if (!first_seg) block_barrier();   // every wave is done with the previous segment's LDS
    }
    seg_pos = SK ? (int64_t)blk * blk_tiles + t1 : seg_end;
    // the segment's key tiles [t0, t1) as if they were all the keys (non-causal when t0 > 0)
    const int nk = SK ? min(a.nkeys - t0 * BN, (t1 - t0) * BN) : a.nkeys;
    const int head = blk / nqb, qblk = blk - head * nqb;
    const int hk = head / a.G;
    const int row0 = qblk * PBM, wrow0 = row0 + wave * 64;
    const int last_row = min(row0 + PBM, a.W) - 1;
    int ntiles = (nk + BN - 1) / BN;
    if (a.causal) ntiles = min(ntiles, (a.p0 + last_row) / BN + 1);
    const uint16_t* kbase = a.k + (int64_t)hk * a.k_hs + (int64_t)t0 * BN * a.k_rs;
    const uint16_t* vbase = a.v + (int64_t)hk * a.v_hs + (int64_t)t0 * PTILE;

    // ---- ring loads: load j of a tile fills rows 4i..4i+3 (K, V rows) or dim rows 8i..8i+7 (V^T), i = wave + PW j, by
    // buffer_load_dwordx4 ... lds from a per-tile descriptor (SGPRs) and a constant per-lane byte offset. The
    // descriptor's record count ends at the last valid key row, so rows past nkeys read as zeros (masked keys; their V
    // rows meet P = 0). A load for a tile past the last one reads nothing (record count 0) into a dummy LDS area, so
    // every step issues the same loads and waits the same counts.
    __shared__ __attribute__((aligned(1024))) uint16_t Dummy[PTILE];
    const int lrow = lane >> 4, lchunk = lane & 15;
    uint32_t koff[PLOADS], voff[PLOADS];
#pragma unroll
    for (int j = 0; j < PLOADS; ++j) {
        const int r = 4 * (wave + PW * j) + lrow;
        koff[j] = 2u * (uint32_t)(r * a.k_rs + 8 * (lchunk ^ (r & 15)));
        if constexpr (VT) {
            const int d = 8 * (wave + PW * j) + (lane >> 3);
            voff[j] = 2u * (uint32_t)(d * BN + 8 * ((lane & 7) ^ ((d >> 1) & 7)));
        } else {
            voff[j] = 2u * (uint32_t)(r * a.v_rs + 8 * (lchunk ^ (lrow << 2)));
        }
    }
    const uint32_t kr_lds = lds_addr(Kr), vr_lds = lds_addr(Vr), dummy_lds = lds_addr(Dummy);
    // Descriptors of tile t of a [rows][row_elems] bf16 array (row stride rs elements). The tiles are loaded in order,
    // so the base address advances by one tile per call. The record count (bytes from the base) is unlimited for a
    // whole tile, ends at the last valid key row for the last tile, and is 0 past it.
    struct TileStream {
        uint64_t addr, step;
        uint32_t last_rec;
    };
    auto rows_stream = [&](const uint16_t* base, int64_t rs) __attribute__((always_inline)) {
        const int64_t last = (int64_t)(nk - 1 - (ntiles - 1) * BN) * rs * 2 + 2 * D;
        return TileStream{(uint64_t)(uintptr_t)base, (uint64_t)(BN * rs * 2),
                          (uint32_t)(last < 0xffffffffLL ? last : 0xffffffffLL)};
    };
    auto next_rsrc = [&](TileStream& ts, int t) __attribute__((always_inline)) {
        const uint64_t addr = ts.addr;
        ts.addr += ts.step;
        const uint32_t rec = t < ntiles - 1 ? 0xffffffffu : t == ntiles - 1 ? ts.last_rec : 0u;
        return u32x4{(uint32_t)addr, (uint32_t)(addr >> 32) & 0xffffu, rec, 0x00020000u};
    };
    TileStream kst = rows_stream(kbase, a.k_rs);
    // packed V^T tiles are whole (zero past nkeys)
    TileStream vst = VT ? TileStream{(uint64_t)(uintptr_t)vbase, 2u * PTILE, 2u * PTILE} : rows_stream(vbase, a.v_rs);
    // this wave's LDS base for tile t of a ring (load j adds j * 4 KB); past the last tile, the dummy area
    const uint32_t wave_lds = (uint32_t)(2 * wave * 512);
    auto lds_dst = [&](uint32_t ring, int t) __attribute__((always_inline)) {
        return (t < ntiles ? ring + (uint32_t)(2 * (t % PNS) * PTILE) : dummy_lds) + wave_lds;
    };
    auto k_rsrc = [&](int t) __attribute__((always_inline)) { return next_rsrc(kst, t); };
    auto v_rsrc = [&](int t) __attribute__((always_inline)) { return next_rsrc(vst, t); };
    // load j of K / V tile t, from its descriptor and LDS base
    auto dma_k = [&](const u32x4& rs, uint32_t dst, int j) __attribute__((always_inline)) {
        dma16_buf(rs, koff[j], dst + (uint32_t)(2 * PW * 512 * j));
    };
    auto dma_v = [&](const u32x4& rs, uint32_t dst, int j) __attribute__((always_inline)) {
        dma16_buf(rs, voff[j], dst + (uint32_t)(2 * PW * 512 * j));
    };

    // ---- prologue loads: K(0), then the queries, then the rest of the ring (K(1), V(0), V(1), K(2), K(3)). The
    // queries' loads are waited for with vmcnt counts that also cover every earlier load: only K(0), which S(0) needs
    // next, is issued before them; the rest of the ring lands while S(0) and the first P are computed.
    {
        const u32x4 rs = k_rsrc(0);
        const uint32_t dst = lds_dst(kr_lds, 0);
#pragma unroll
        for (int j = 0; j < PLOADS; ++j) dma_k(rs, dst, j);
    }
    bf16x8 qa[2][8];   // AGPR-resident B operands of S^T = K Q^T
    {
        bf16x8 qv[8];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            const int qrow = wrow0 + 32 * nb + n;
            if constexpr (QK == QK_PLAIN)
                load_q_plain(a, qrow, head, hf, qv);
            else
                load_q_fused<QK>(a, qrow, head, hf, qv, a.c);
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) asm volatile("; q -> agpr" : "=a"(qa[nb][ks]) : "0"(qv[ks]));
            fence_q(qa[nb]);   // the AGPR writes above land before the first MFMA reads them
        }
    }
    // K(1), V(0), V(1), K(2), K(3): the step-closing waits count on V(1) being older than K(3)
#pragma unroll
    for (int i = 0; i < 5; ++i) {
        const bool is_v = i == 1 || i == 2;
        const int tt = i == 0 ? 1 : i - 1;
        const u32x4 rs = is_v ? v_rsrc(tt) : k_rsrc(tt);
        const uint32_t dst = lds_dst(is_v ? vr_lds : kr_lds, tt);
#pragma unroll
        for (int j = 0; j < PLOADS; ++j) {
            if (is_v) dma_v(rs, dst, j);
            else dma_k(rs, dst, j);
        }
    }

    // ---- per-lane LDS byte offsets. K fragment (k-step ks, 32-key block mb) of a tile: row 32 mb + key_perm(n),
    // chunk (2 ks + hf) ^ (row & 15); with the row a multiple of 256 bytes that is lane_k ^ (32 ks) + 8192 mb.
    // Packed V^T fragment (16-key step kk, 32-dim block db): dim row 32 db + n, chunk (2 kk + hf) ^ ((n >> 1) & 7),
    // i.e. lane_v ^ (32 kk) + 4096 db.
    const int pr = key_perm(n);
    const uint32_t lane_k = (uint32_t)(pr * 256 + 16 * (hf ^ (pr & 15)));
    const uint32_t lane_v = (uint32_t)(n * 128 + 16 * (hf ^ ((n >> 1) & 7)));
    const int g = lane >> 4, sl = lane & 15;
    int vtr[4];   // V rows read transposed (plain path)
#pragma unroll
    for (int db = 0; db < 4; ++db) {
        const int chunk = 4 * (db ^ (sl >> 2)) + 2 * (g & 1) + ((sl & 3) >> 1);
        vtr[db] = (8 * (g >> 1) + (sl >> 2)) * D + 8 * chunk + 4 * (sl & 1);
    }
    typedef __attribute__((address_space(3))) const bf16x8 lds_bf16x8;
    // kslot / vslot: LDS byte address of the tile's ring slot
    auto kfrag = [&](uint32_t kslot, int mb, int ks) __attribute__((always_inline)) -> bf16x8 {
        return *(lds_bf16x8*)(uintptr_t)(kslot + (lane_k ^ (uint32_t)(32 * ks)) + 8192 * mb);
    };
    auto vfrag = [&](uint32_t vslot, int i) __attribute__((always_inline)) -> bf16x8 {   // i = 4 kk + db
        const int kk = i >> 2, db = i & 3;
        if constexpr (VT) {
            return *(lds_bf16x8*)(uintptr_t)(vslot + (lane_v ^ (uint32_t)(32 * kk)) + 4096 * db);
        } else {
            const uint32_t p0 = vslot + 2 * (vtr[db] + (16 * kk) * D);
            const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(uintptr_t)p0);
            const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(uintptr_t)(p0 + 8 * D));
            return __builtin_shufflevector(__builtin_bit_cast(bf16x4, lo), __builtin_bit_cast(bf16x4, hi), 0, 1, 2, 3,
                                           4, 5, 6, 7);
        }
    };
    auto kslot_of = [&](int t) __attribute__((always_inline)) { return kr_lds + (uint32_t)((t % PNS) * PTILE * 2); };
    auto vslot_of = [&](int t) __attribute__((always_inline)) { return vr_lds + (uint32_t)((t % PNS) * PTILE * 2); };

    LR_WAIT_VMCNT(5 * PLOADS);   // K(0) and the queries have landed; K(1..3), V(0..1) may still be in flight
    block_barrier();

    // ---- S(0) = K(0) Q^T
    f32x16 s[2][2];   // [query block][32-key block]
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const bf16x8 kf = kfrag(kslot_of(0), mb, ks);
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                if (ks == 0) mfma_qk0(s[nb][mb], kf, qa[nb][0]);
                else mfma_qk(s[nb][mb], kf, qa[nb][ks]);
            }
        }

    const float c = a.c;
    // the tiles from t_mask on have keys past nkeys or, causal, past some query of this wave
    int t_mask = nk / BN;
    if (a.causal) t_mask = min(t_mask, (a.p0 + wrow0 - (BN - 1)) >= 0 ? (a.p0 + wrow0 - (BN - 1)) / BN + 1 : 0);
    auto needs_mask = [&](int t) __attribute__((always_inline)) { return t >= t_mask; };
    // Register r of score tile (nb, mb) holds key t BN + 32 mb + 8 hf + c(r), c(r) = 16 (r >> 3) + (r & 7), of query
    // row wrow0 + 32 nb + n. It is valid iff c(r) < lim: the compile-time c(r) against one lane value per tile.
    auto mask_block = [&](int t, int mb) __attribute__((always_inline)) {
        const int key0 = t * BN + 32 * mb + 8 * hf;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            int lim = nk - key0;
            if (a.causal) lim = min(lim, a.p0 + wrow0 + 32 * nb + n - key0 + 1);
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if (!(16 * (r >> 3) + (r & 7) < lim)) s[nb][mb][r] = -INFINITY;
        }
    };
    auto block_max = [&](int nb, int mb) __attribute__((always_inline)) {
        float m = fmaxf(s[nb][mb][0], s[nb][mb][1]);
#pragma unroll
        for (int r = 2; r < 16; ++r) m = fmaxf(m, s[nb][mb][r]);
        return m;
    };

    // ---- the reference: ceil of tile 0's exact max (the exp2 domain), fixed for the whole call. Later tiles' P are
    // exp2(s - m) with no running max: exact as long as they stay finite, which the epilogue verifies
    fence_s(s);
    if (needs_mask(0)) {
        mask_block(0, 0);
        mask_block(0, 1);
    }
    float m_used[2], ls[2] = {0.0f, 0.0f};
    f32x16 negm[2];   // FOLD: -m in every slot, the initial accumulator of the score MFMAs
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        float mx = wave_pair_max(fmaxf(block_max(nb, 0), block_max(nb, 1)));
        if constexpr (!FOLD) mx *= c;
        m_used[nb] = mx > -INFINITY ? ceilf(mx) : 0.0f;
        negm[nb] = f32x16{} - m_used[nb];
        if constexpr (FOLD) {
            s[nb][0] -= m_used[nb];
            s[nb][1] -= m_used[nb];
        }
    }
    fence_negm(negm);
    f32x16 o[2][4];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int db = 0; db < 4; ++db) o[nb][db] = f32x16{};
    LR_WAIT_VMCNT(4 * PLOADS);   // K(1) has landed (step 0 reads it from its first slot)
    block_barrier();             // ... in every wave; and every wave is done with K slot 0 before step 0 refills it

    u32x4 pA[2][4], pB[2][4];   // P double buffer: packed bf16 pairs, [query block][16-key step kk][j]

    // P word w (0..15) of key block mb: (nb, kk, j) = (w / 8, 2 mb + (w / 4) % 2, w % 4), keys 16 kk + 8 hf + 2 j, +1
    // of the tile, from score registers r, r + 1 of tile (nb, mb), r = 8 ((w / 4) % 2) + 2 j. A word takes three
    // stages in consecutive slots, so that no instruction waits on the one before it: E (two exp2), C (bf16 pack into
    // the P buffer, and the pair's fp32 sum), D (the pair sum into the row sum). The row sum is over the fp32 P, as
    // the reference's (attention.cu:403-407); the PV product takes P rounded to bf16 (attention.cu:418-424).
    float e0, e1, es;
    auto stage_e = [&](int mb, int w) __attribute__((always_inline)) {
        const int nb = w >> 3, r = 8 * ((w >> 2) & 1) + 2 * (w & 3);
        const float x0 = s[nb][mb][r], x1 = s[nb][mb][r + 1];
        e0 = __builtin_amdgcn_exp2f(FOLD ? x0 : fmaf(x0, c, -m_used[nb]));
        e1 = __builtin_amdgcn_exp2f(FOLD ? x1 : fmaf(x1, c, -m_used[nb]));
        asm volatile("" ::"v"(e0), "v"(e1));   // computed in this slot, not sunk towards their use
    };
    auto stage_c = [&](u32x4 (&p)[2][4], int mb, int w) __attribute__((always_inline)) {
        const uint32_t x = pack_bf16x2(e0, e1);
        es = e0 + e1;
        asm volatile("" ::"v"(x), "v"(es));
        p[w >> 3][2 * mb + ((w >> 2) & 1)][w & 3] = x;
    };
    auto stage_d = [&](int w) __attribute__((always_inline)) {
        const int nb = w >> 3;
        ls[nb] += es;
        asm volatile("" ::"v"(ls[nb]));
    };
    auto pv_operand = [&](const u32x4 (&p)[2][4], int nb, int kk) __attribute__((always_inline)) {
        return __builtin_bit_cast(bf16x8, p[nb][kk]);
    };
    // QK MFMA k-step ks of score tile (nb, mb) of the next tile
    auto qk = [&](int nb, int mb, int ks, const bf16x8& kf) __attribute__((always_inline)) {
        if (ks == 0) {
            if constexpr (FOLD) mfma_qk_c(s[nb][mb], kf, qa[nb][0], negm[nb]);
            else mfma_qk0(s[nb][mb], kf, qa[nb][0]);
        } else {
            mfma_qk(s[nb][mb], kf, qa[nb][ks]);
        }
    };

    // P(0) of key block 0, words 0-10 (the steps carry the rest)
#pragma unroll
    for (int w = 0; w < 11; ++w) {
        stage_e(0, w);
        stage_c(pA, 0, w);
        stage_d(w);
    }

    bf16x8 fr[4];   // fragment ring, read 3 fragments ahead
    // fragment f of a step: V0-V11, K(block 0, ks 0-7), V12-V15, K(block 1, ks 0-7)
    auto frag_is_v = [](int f) { return f < 12 || (f >= 20 && f < 24); };
    auto frag_of = [&](uint32_t kt, uint32_t vt, int f) __attribute__((always_inline)) -> bf16x8 {
        if (f < 12) return vfrag(vt, f);
        if (f < 20) return kfrag(kt, 0, f - 12);
        if (f < 24) return vfrag(vt, f - 8);
        return kfrag(kt, 1, f - 24);
    };

    // the ring refill of step t, one load per slot 3, 7, ..., 31: V(t+2) loads 0-3, then K(t+4) loads 0-3. Their
    // descriptors are formed in slots 0 and 2, under the MFMAs, rather than before the step's first MFMA.
    struct Refill {
        u32x4 krs, vrs;
        uint32_t kdst, vdst;
    };
    auto refill_slot = [&](Refill& rf, int t, int sl2) __attribute__((always_inline)) {
        if (sl2 == 0) {
            rf.vrs = v_rsrc(t + 2);
            rf.vdst = lds_dst(vr_lds, t + 2);
        } else if (sl2 == 2) {
            rf.krs = k_rsrc(t + PNS);
            rf.kdst = lds_dst(kr_lds, t + PNS);
        }
        if ((sl2 & 3) != 3 || sl2 >= 32) return;
        const int j = sl2 >> 2;
        if (j < 4) dma_v(rf.vrs, rf.vdst, j);
        else dma_k(rf.krs, rf.kdst, j - 4);
    };
    // end of step t: wait for this wave's loads up to V(t+1) (issued in step t-1; only K(t+3) and this step's loads may
    // stay in flight), read the next step's first fragments (V(t), resident in every wave since the previous barrier),
    // barrier. Step t+1 reads K(t+2) and V(t), both issued in step t-2, so the K loads get two steps to land.
    auto close_step = [&](int t) __attribute__((always_inline)) {
        LR_WAIT_VMCNT(3 * PLOADS);
        const uint32_t vt = vslot_of(t);
        fr[0] = vfrag(vt, 0);
        fr[1] = vfrag(vt, 1);
        fr[2] = vfrag(vt, 2);
        block_barrier();
    };

    // ---- step t: PV(t-1) (none in the first step), the rest of P(t), S(t+1), and P(t+1) of key block 0 as soon as
    // its scores are out of the MFMA pipe. One uninterrupted run of 64 slots:
    //   slots  0-23  PV fragments V0-V11   | P(t) key block 0, words 11-15 (E in slots 0, 2, ..., 8)
    //   slots 24-39  S(t+1) key block 0    | P(t) key block 1, words 0-15 (E in slots 10, 12, ..., 40)
    //   slots 40-47  PV fragments V12-V15  | (slot 41) mask S(t+1) key block 0 if the tile needs it
    //   slots 48-63  S(t+1) key block 1    | P(t+1) key block 0, words 0-10 (E in slots 42, 44, ..., 62)
    // A word's C and D stages follow its E one and two slots later; word 10 of P(t+1)'s D runs in slot 0 of step t+1.
    // Ring loads in slots 3, 7, ..., 31. For the last tile, S(t+1) is past every key, so P(t+1) is masked to zeros.
    auto step = [&](int t, u32x4 (&pc)[2][4], u32x4 (&pn)[2][4], auto first_tag) __attribute__((always_inline)) {
        constexpr bool FIRST = decltype(first_tag)::value;
        if (!FIRST && needs_mask(t)) {   // key block 0 of S(t) was masked in the previous step
            fence_s(s);
            mask_block(t, 1);
        }
        const uint32_t kt = kslot_of(t + 1);
        const uint32_t vt = vslot_of(t - 1);
        Refill rf;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int sl2 = 0; sl2 < 64; ++sl2) {
            const int f = sl2 >> 1, nb = sl2 & 1;
            if (nb == 0 && f + 3 < 32 && !(FIRST && frag_is_v(f + 3))) fr[(f + 3) & 3] = frag_of(kt, vt, f + 3);
            if (frag_is_v(f)) {
                if constexpr (!FIRST) {
                    const int i = f < 12 ? f : f - 8;   // V fragment 4 kk + db
                    mfma_pv(o[nb][i & 3], fr[f & 3], pv_operand(pn, nb, i >> 2));
                }
            } else {
                const int mb = f < 20 ? 0 : 1, ks = f < 20 ? f - 12 : f - 24;
                qk(nb, mb, ks, fr[f & 3]);
            }
            // the word whose stage X runs in this slot had its E stage in slot sl2 - X
            auto word_at = [&](int e_slot, auto&& fn) __attribute__((always_inline)) {
                if (e_slot < 0 || (e_slot & 1)) return;
                if (e_slot <= 8) fn(pc, 0, 11 + e_slot / 2);
                else if (e_slot <= 40) fn(pc, 1, (e_slot - 10) / 2);
                else fn(pn, 0, (e_slot - 42) / 2);
            };
            if (!FIRST && sl2 == 0) stage_d(10);   // D of the last word the previous step started
            word_at(sl2 - 2, [&](const u32x4 (&)[2][4], int, int w) __attribute__((always_inline)) { stage_d(w); });
            word_at(sl2 - 1, [&](u32x4 (&p)[2][4], int mb, int w) __attribute__((always_inline)) { stage_c(p, mb, w); });
            word_at(sl2, [&](u32x4 (&)[2][4], int mb, int w) __attribute__((always_inline)) { stage_e(mb, w); });
            if (sl2 == 41) {
                __builtin_amdgcn_sched_barrier(0);
                if (needs_mask(t + 1)) {
                    fence_s(s);
                    mask_block(t + 1, 0);
                }
            }
            refill_slot(rf, t, sl2);
            __builtin_amdgcn_sched_barrier(0);
        }
        close_step(t);
    };

    step(0, pA, pB, BoolTag<true>{});
    int t = 1;
    for (; t + 1 < ntiles; t += 2) {
        step(t, pB, pA, BoolTag<false>{});
        step(t + 1, pA, pB, BoolTag<false>{});
    }
    if (t < ntiles) step(t, pB, pA, BoolTag<false>{});

    // ---- PV of the last tile (its first three fragments are in the ring)
    auto last_pv = [&](const u32x4 (&p)[2][4]) __attribute__((always_inline)) {
        const uint32_t vt = vslot_of(ntiles - 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int sl2 = 0; sl2 < 32; ++sl2) {
            const int f = sl2 >> 1, nb = sl2 & 1;
            if (nb == 0 && f + 3 < 16) fr[(f + 3) & 3] = vfrag(vt, f + 3);
            mfma_pv(o[nb][f & 3], fr[f & 3], pv_operand(p, nb, f >> 2));
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    if ((ntiles - 1) & 1) last_pv(pB);
    else last_pv(pA);
    LR_WAIT_VMCNT(0);   // the last steps' loads (into the dummy area) have landed before the workgroup ends
    fence_o(o);

    if constexpr (SK) {
        if (t0 > 0 || t1 < blk_tiles) {   // a part of a cut block: store the partial, go on with the next segment
            const int slot = t0 > 0 ? 2 * logical + 1 : 2 * (logical + 1);
            float* part = a.sk_part + (size_t)slot * (PW * SK_WAVE_FLOATS) + wave * SK_WAVE_FLOATS;
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                for (int db = 0; db < 4; ++db)
#pragma unroll
                    for (int gg = 0; gg < 4; ++gg) {
                        const float4 v = {o[nb][db][4 * gg], o[nb][db][4 * gg + 1], o[nb][db][4 * gg + 2],
                                          o[nb][db][4 * gg + 3]};
                        *reinterpret_cast<float4*>(part + 4 * (((nb * 4 + db) * 4 + gg) * 64 + lane)) = v;
                    }
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                part[SK_ML + (2 * nb) * 64 + lane] = m_used[nb];
                part[SK_ML + (2 * nb + 1) * 64 + lane] = ls[nb];
            }
            continue;
        }
    }

    bool overflow = false;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        const int qrow = wrow0 + 32 * nb + n;
        const float l = wave_pair_sum(ls[nb]);
        const float inv = 1.0f / l;
        bool bad = !__builtin_isfinite(l);
        if (qrow < a.W) {
            uint16_t* dst = a.out + (int64_t)qrow * a.o_rs + head * D + 4 * hf;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int gg = 0; gg < 4; ++gg) {
                    const float y0 = o[nb][db][4 * gg] * inv, y1 = o[nb][db][4 * gg + 1] * inv;
                    const float y2 = o[nb][db][4 * gg + 2] * inv, y3 = o[nb][db][4 * gg + 3] * inv;
                    bad = bad || !__builtin_isfinite(y0) || !__builtin_isfinite(y1) || !__builtin_isfinite(y2) ||
                          !__builtin_isfinite(y3);
                    u32x2 w;
                    w[0] = pack_bf16x2(y0, y1);
                    w[1] = pack_bf16x2(y2, y3);
                    *reinterpret_cast<u32x2*>(dst + 32 * db + 8 * gg) = w;
                }
        }
        overflow = overflow || bad;
    }
    if (__builtin_amdgcn_ballot_w64(overflow) && lane == 0 && wrow0 < a.W)
        a.out[(int64_t)wrow0 * a.o_rs + head * D] = 0x7fc0;   // bf16 quiet NaN
    }   // segments
}

// Merge the two parts of the block cut at the start of stream-K range c = blockIdx.x + 1 (none when that range starts at a
// block boundary) and write its rows: one wave per 64-query quarter, each lane the (row, dims) set its wave's lane held
// in the attention kernel.
__global__ __launch_bounds__(PW * 64) void attn_sk_combine_kernel(AttnArgs a, int blk_tiles) {
    const int c = blockIdx.x + 1, nwg = gridDim.x + 1;
    const int nqb = (a.W + PBM - 1) / PBM;
    const SkCut cut = sk_cut(c, nqb * a.H, blk_tiles, nwg);
    if (cut.t == 0) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n = lane & 31, hf = lane >> 5;
    const int head = cut.blk / nqb, qblk = cut.blk - head * nqb;
    const int wrow0 = qblk * PBM + wave * 64;
    const float* ph = a.sk_part + (size_t)(2 * c) * (PW * SK_WAVE_FLOATS) + wave * SK_WAVE_FLOATS;
    const float* pt = ph + PW * SK_WAVE_FLOATS;
    bool overflow = false;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        const float mh = ph[SK_ML + (2 * nb) * 64 + lane], lh = ph[SK_ML + (2 * nb + 1) * 64 + lane];
        const float mt = pt[SK_ML + (2 * nb) * 64 + lane], lt = pt[SK_ML + (2 * nb + 1) * 64 + lane];
        const float mn = fmaxf(mh, mt);
        const float sh = __builtin_amdgcn_exp2f(mh - mn), st = __builtin_amdgcn_exp2f(mt - mn);
        const float l = wave_pair_sum(lh * sh + lt * st);
        const float inv = 1.0f / l;
        bool bad = !__builtin_isfinite(l);
        const int qrow = wrow0 + 32 * nb + n;
        uint16_t* dst = a.out + (int64_t)qrow * a.o_rs + head * D + 4 * hf;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int gg = 0; gg < 4; ++gg) {
                const int i = 4 * (((nb * 4 + db) * 4 + gg) * 64 + lane);
                const float4 x = *reinterpret_cast<const float4*>(ph + i);
                const float4 y = *reinterpret_cast<const float4*>(pt + i);
                const float y0 = (x.x * sh + y.x * st) * inv, y1 = (x.y * sh + y.y * st) * inv;
                const float y2 = (x.z * sh + y.z * st) * inv, y3 = (x.w * sh + y.w * st) * inv;
                bad = bad || !__builtin_isfinite(y0) || !__builtin_isfinite(y1) || !__builtin_isfinite(y2) ||
                      !__builtin_isfinite(y3);
                if (qrow < a.W) {
                    u32x2 w;
                    w[0] = pack_bf16x2(y0, y1);
                    w[1] = pack_bf16x2(y2, y3);
                    *reinterpret_cast<u32x2*>(dst + 32 * db + 8 * gg) = w;
                }
            }
        overflow = overflow || (bad && qrow < a.W);
    }
    if (__builtin_amdgcn_ballot_w64(overflow) && lane == 0 && wrow0 < a.W)
        a.out[(int64_t)wrow0 * a.o_rs + head * D] = 0x7fc0;   // marked for the running-max launch
}

// CUs of the current device (cached per device), capped at SK_MAX_WG
int sk_workgroups() {
    static int cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) return 0;
        cus[dev] = min(n, SK_MAX_WG);
    }
    return cus[dev];
}

template <int QK, bool VT>
hipError_t launch_pair_t(const AttnArgs& a, hipStream_t stream) {
    const int64_t nqb = (a.W + PBM - 1) / PBM;
    const int64_t blocks = nqb * a.H;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    if constexpr (VT) {
        // stream-K where whole blocks would leave more than 3% of the last round idle, given the partials area and at
        // least one block per workgroup
        const int nwg = a.sk_part && !a.causal ? sk_workgroups() : 0;
        if (nwg > 1 && blocks >= nwg) {
            const int64_t rounds = (blocks + nwg - 1) / nwg;
            if (blocks * 100 < rounds * nwg * 97) {
                hipLaunchKernelGGL((attn_pair_kernel<QK, VT, true>), dim3((unsigned)nwg), dim3(PW * 64), 0, stream, a);
                const hipError_t e = hipGetLastError();
                if (e != hipSuccess) return e;
                hipLaunchKernelGGL(attn_sk_combine_kernel, dim3((unsigned)(nwg - 1)), dim3(PW * 64), 0, stream, a,
                                   (int)((a.nkeys + BN - 1) / BN));
                return hipGetLastError();
            }
        }
    }
    hipLaunchKernelGGL((attn_pair_kernel<QK, VT, false>), dim3((unsigned)blocks), dim3(PW * 64), 0, stream, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_pair(const AttnArgs& a, int qk, bool v_t, hipStream_t stream) {
    if (v_t) {
        switch (qk) {
            case TABLE_NONE: return launch_pair_t<TABLE_NONE, true>(a, stream);
            case TABLE_COSSIN_F32: return launch_pair_t<TABLE_COSSIN_F32, true>(a, stream);
            case TABLE_MAT2_BF16: return launch_pair_t<TABLE_MAT2_BF16, true>(a, stream);
            case TABLE_MAT2_F32: return launch_pair_t<TABLE_MAT2_F32, true>(a, stream);
            default: return hipErrorInvalidValue;
        }
    }
    if (qk == QK_PLAIN) return launch_pair_t<QK_PLAIN, false>(a, stream);
    return hipErrorInvalidValue;
}

}  // namespace lr
