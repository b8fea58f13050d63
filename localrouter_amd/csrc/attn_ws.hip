// Warp-specialised flash attention for gfx950 ("ws" kernel): two waves per SIMD, one computing scores and softmax,
// the other the PV products. bf16 in, fp32 MFMA accumulation and softmax, bf16 out. Same semantics as
// attn_pair.hip (kernels/cuda/qwen_image/attention.cu:253-444 as launched by ops_launch.zig:163-172; P rounded to
// bf16 for the PV product, attention.cu:418-424; the row sum over the fp32 P, attention.cu:403-407), for the fused
// and prepared calls (queries normalised and rotated in registers, keys prepared, values as packed V^T tiles),
// non-causal.
//
// Why. With one wave per SIMD (attn_pair.hip) every softmax VALU instruction sits in the same in-order stream as the
// MFMAs, and a step of 64 MFMAs (2,048 cycles of matrix work) takes ~3,600 cycles. Here each SIMD runs a pair:
//   wave A (waves 0-3): S(t+1) = K(t+1) Q^T (32 MFMAs a step) and the softmax of S (exp2, bf16 pack, row sums);
//                       it writes P(t) to LDS.
//   wave B (waves 4-7): O += V(t-1)^T P(t-1) (32 MFMAs a step) with P read back from LDS.
// The SIMD issues B's MFMAs while A works on the VALU, and the other way round. Each pair owns 64 queries (two
// 32-query blocks); each K or V^T fragment read from LDS feeds two MFMAs. All state is in VGPRs (A: Q 64, S 64,
// -m 16, fragments 16; B: O 128, P 32, fragments 16): the kernel fits 256 registers a wave.
//
// Per step t (two workgroup barriers):
//   A: [G0] S(t+1) key block 0 (16 MFMAs) | P(t) key block 1: one word (two keys of one query) per slot, in three
//      stages one slot apart (exp2 | pack + pair sum | row sum), 4-word groups written to the LDS P buffer of t
//      [mid barrier] (if the tile needs it, S(t+1) key block 0 masked)
//      [G1] S(t+1) key block 1 (16 MFMAs) | P(t+1) key block 0, into the P buffer of t+1
//      K(t+3) loads in G0 (3-stage K ring).   [end barrier]
//   B: P(t-1) operands read from LDS at the step start; [slots 0-15] PV fragments V0-V7 | [mid barrier: B has read
//      the P buffer that A's G1 overwrites] | [slots 16-31] PV fragments V8-V15; V(t) loads (2-stage V^T ring).
//      [end barrier]
// Step 0 has no PV; after the last step B runs PV(ntiles-1). P(0) of key block 0 is computed in the prologue.
//
// Softmax against a fixed reference per query (the ceil of its exact maximum over the first key tile, exp2 domain),
// folded into the score MFMAs, as in attn_pair.hip: exact while every P, the row sums and O stay finite. The epilogue
// checks l and O; a wave pair with a row that is not finite marks its first row with a NaN, and the running-max
// kernel of attn_fwd.hip, launched next over the same 256-query blocks, recomputes exactly the marked blocks.
#include "lr_common.h"
#include "lr_kernels.h"

namespace lr {

namespace {

#include "attn_common.inc"

// One 16-byte-per-lane ring load, buffer -> LDS (as attn_pair.hip): lane l reads 16 bytes at descriptor base + voff
// (zeros past the record count) and they land at LDS byte address lds + 16 l.
// (voff per lane, soff wave-uniform)
__device__ __forceinline__ void ws_dma(u32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rsrc),
                 "s"(soff), "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory");
}

// O += V^T P through the builtin (the compiler keeps O in AGPRs and inserts the hazard waits of its copies).
__device__ __forceinline__ void ws_mfma(f32x16& d, const bf16x8& a, const bf16x8& b) {
    d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, d, 0, 0, 0);
}
// S = K Q^T + c, S += K Q^T as inline asm: S in VGPRs (the softmax reads them), Q in AGPRs. The compiler does not see
// these as MFMAs: every VALU access to S is many MFMAs later or behind ws_fence_s.
__device__ __forceinline__ void ws_qk_c(f32x16& d, const bf16x8& k, const bf16x8& q, const f32x16& c) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %3" : "=&v"(d) : "v"(k), "a"(q), "v"(c));
}
__device__ __forceinline__ void ws_qk(f32x16& d, const bf16x8& k, const bf16x8& q) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(k), "a"(q));
}
// wait states (more than an MFMA result needs before a VALU access) whose asm takes the protected registers
#define WS_NOP48 "s_nop 15\n\ts_nop 15\n\ts_nop 15"
__device__ __forceinline__ void ws_fence_s(f32x16 (&s)[2][2]) {
    asm volatile(WS_NOP48 : "+v"(s[0][0]), "+v"(s[0][1]), "+v"(s[1][0]), "+v"(s[1][1]));
}
__device__ __forceinline__ void ws_fence_s0(f32x16 (&s)[2][2]) {
    asm volatile("s_nop 15\n\ts_nop 3" : "+v"(s[0][0]), "+v"(s[1][0]));
}
__device__ __forceinline__ void ws_fence_q(bf16x8 (&q)[8]) {
    asm volatile(WS_NOP48 : "+a"(q[0]), "+a"(q[1]), "+a"(q[2]), "+a"(q[3]), "+a"(q[4]), "+a"(q[5]), "+a"(q[6]),
                 "+a"(q[7]));
}
__device__ __forceinline__ void ws_fence_negm(f32x16& m) { asm volatile(WS_NOP48 : "+v"(m)); }

#define LR_WAIT_LGKM0() asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory")

constexpr int WS_PAIRS = 4;                 // SIMDs, wave pairs per workgroup
constexpr int WS_BM = 64 * WS_PAIRS;        // queries per workgroup
constexpr int WS_KNS = 3;                   // K ring stages
constexpr int WS_VNS = 2;                   // V^T ring stages
constexpr int WS_TILE = BN * D;             // elements per K or V^T tile
constexpr int WS_LOADS = BN / 4 / WS_PAIRS; // 1 KB direct loads per wave per tile (A: K, B: V^T)
constexpr int WS_PBUF = 2 * 4 * 1024;       // bytes of one P buffer of a pair: [nb 2][kk 4][64 lanes x 16 B]

template <int QK>
__global__ __launch_bounds__(2 * WS_PAIRS * 64, 1) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_ws_kernel(
    AttnArgs a) {
    __shared__ __attribute__((aligned(1024))) uint16_t Kr[WS_KNS * WS_TILE];
    __shared__ __attribute__((aligned(1024))) uint16_t Vr[WS_VNS * WS_TILE];
    __shared__ __attribute__((aligned(1024))) uint32_t Pb[WS_PAIRS * 2 * WS_PBUF / 4];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool is_a = wave < WS_PAIRS;
    const int pair = wave & (WS_PAIRS - 1);
    const int n = lane & 31, hf = lane >> 5;

    // XCD-aware mapping, as attn_pair.hip
    const int nwg = gridDim.x, b = blockIdx.x;
    const int per = nwg >> 3, rem = nwg & 7, xcd = b & 7, idx = b >> 3;
    const int logical = xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
    const int nqb = (a.W + WS_BM - 1) / WS_BM;
    const int head = logical / nqb, qblk = logical - head * nqb;
    const int hk = head / a.G;
    const int row0 = qblk * WS_BM, wrow0 = row0 + pair * 64;
    const int ntiles = (a.nkeys + BN - 1) / BN;
    const uint16_t* kbase = a.k + (int64_t)hk * a.k_hs;
    const uint16_t* vbase = a.v + (int64_t)hk * a.v_hs;

    const uint32_t kr_lds = lds_addr(Kr), vr_lds = lds_addr(Vr);
    const uint32_t pb_lds = lds_addr(Pb) + (uint32_t)(pair * 2 * WS_PBUF);
    auto kslot = [&](int t) __attribute__((always_inline)) { return kr_lds + (uint32_t)((t % WS_KNS) * WS_TILE * 2); };
    auto vslot = [&](int t) __attribute__((always_inline)) { return vr_lds + (uint32_t)((t % WS_VNS) * WS_TILE * 2); };
    // P buffer of tile t, operand (nb, kk): this lane's 16 bytes
    auto p_addr = [&](int t, int nb, int kk) __attribute__((always_inline)) {
        return pb_lds + (uint32_t)((t & 1) * WS_PBUF + (nb * 4 + kk) * 1024 + lane * 16);
    };

    // ---- ring loads (A: K tiles, B: V^T tiles), descriptors advancing one tile per load, as attn_pair.hip
    const int lw = pair;   // the wave's index among the loaders of its kind
    // Load j covers rows (or V^T dim rows) 16 j further than load 0, with the same swizzle (r & 15 and (d >> 1) & 7
    // do not change by 16 rows): one per-lane offset, plus a wave-uniform one per load.
    const int lrow = lane >> 4, lchunk = lane & 15;
    uint32_t loff, lstep;
    if (is_a) {
        const int r = 4 * lw + lrow;
        loff = 2u * (uint32_t)(r * a.k_rs + 8 * (lchunk ^ (r & 15)));
        lstep = 2u * (uint32_t)(4 * WS_PAIRS * a.k_rs);
    } else {
        const int d = 8 * lw + (lane >> 3);
        loff = 2u * (uint32_t)(d * BN + 8 * ((lane & 7) ^ ((d >> 1) & 7)));
        lstep = 2u * (uint32_t)(8 * WS_PAIRS * BN);
    }
    struct TileStream {
        uint64_t addr, step;
        uint32_t last_rec;
    };
    TileStream ts;
    if (is_a) {
        const int64_t last = (int64_t)(a.nkeys - 1 - (ntiles - 1) * BN) * a.k_rs * 2 + 2 * D;
        ts = TileStream{(uint64_t)(uintptr_t)kbase, (uint64_t)(BN * a.k_rs * 2),
                        (uint32_t)(last < 0xffffffffLL ? last : 0xffffffffLL)};
    } else {
        ts = TileStream{(uint64_t)(uintptr_t)vbase, 2u * WS_TILE, 2u * WS_TILE};
    }
    auto next_rsrc = [&](int t) __attribute__((always_inline)) {
        const uint64_t addr = ts.addr;
        ts.addr += ts.step;
        const uint32_t rec = t < ntiles - 1 ? 0xffffffffu : t == ntiles - 1 ? ts.last_rec : 0u;
        return u32x4{(uint32_t)addr, (uint32_t)(addr >> 32) & 0xffffu, rec, 0x00020000u};
    };
    const uint32_t wave_lds = (uint32_t)(2 * lw * 512);
    // issue load j of tile t (tiles in order, one descriptor per tile)
    u32x4 cur_rs;
    auto load_tile = [&](int t, int j) __attribute__((always_inline)) {
        if (j == 0) cur_rs = next_rsrc(t);
        const uint32_t dst = (is_a ? kslot(t) : vslot(t)) + wave_lds + (uint32_t)(2 * WS_PAIRS * 512 * j);
        ws_dma(cur_rs, loff, lstep * (uint32_t)j, dst);
    };

    // ---- LDS fragment addresses, as attn_pair.hip
    const int pr = key_perm(n);
    uint32_t lane_k = (uint32_t)(pr * 256 + 16 * (hf ^ (pr & 15)));
    const uint32_t lane_v = (uint32_t)(n * 128 + 16 * (hf ^ ((n >> 1) & 7)));
    typedef __attribute__((address_space(3))) const bf16x8 lds_bf16x8;
    typedef __attribute__((address_space(3))) const u32x4 lds_u32x4;
    typedef __attribute__((address_space(3))) u32x4 lds_u32x4w;
    auto kfrag = [&](uint32_t ks_, int mb, int ks) __attribute__((always_inline)) -> bf16x8 {
        return *(lds_bf16x8*)(uintptr_t)(ks_ + (lane_k ^ (uint32_t)(32 * ks)) + 8192 * mb);
    };
    auto vfrag = [&](uint32_t vs_, int i) __attribute__((always_inline)) -> bf16x8 {   // i = 4 kk + db
        const int kk = i >> 2, db = i & 3;
        return *(lds_bf16x8*)(uintptr_t)(vs_ + (lane_v ^ (uint32_t)(32 * kk)) + 4096 * db);
    };

    const int t_mask = a.nkeys / BN;   // tiles from t_mask on hold keys past nkeys
    auto needs_mask = [&](int t) __attribute__((always_inline)) { return t >= t_mask; };

    if (is_a) {
        // ================================================================ wave A: scores and softmax
        bf16x8 q[2][8];   // AGPR-resident B operands of S^T = K Q^T
#pragma unroll
        for (int j = 0; j < WS_LOADS; ++j) load_tile(0, j);
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            bf16x8 qv[8];
            load_q_fused<QK>(a, wrow0 + 32 * nb + n, head, hf, qv, a.c);
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) asm volatile("; q -> agpr" : "=a"(q[nb][ks]) : "0"(qv[ks]));
            ws_fence_q(q[nb]);
        }
#pragma unroll
        for (int t = 1; t < WS_KNS; ++t)
#pragma unroll
            for (int j = 0; j < WS_LOADS; ++j) load_tile(t, j);
        LR_WAIT_VMCNT(2 * WS_LOADS);   // K(0) and the queries have landed
        block_barrier();               // P1: K(0) in every A wave's share

        f32x16 s[2][2];   // [query block][32-key block]
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                const bf16x8 kf = kfrag(kslot(0), mb, ks);
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
                    if (ks == 0) ws_qk_c(s[nb][mb], kf, q[nb][0], f32x16{});
                    else ws_qk(s[nb][mb], kf, q[nb][ks]);
                }
            }
        ws_fence_s(s);
        auto mask_block = [&](int t, int mb) __attribute__((always_inline)) {
            const int key0 = t * BN + 32 * mb + 8 * hf;
            const int lim = a.nkeys - key0;
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (!(16 * (r >> 3) + (r & 7) < lim)) s[nb][mb][r] = -INFINITY;
        };
        if (needs_mask(0)) {
            mask_block(0, 0);
            mask_block(0, 1);
        }
        // One reference per lane for its two queries (n of each query block): softmax is shift-invariant per row, so
        // any per-row constant is exact while P stays finite and normal; a row whose own maximum lies far below the
        // other's (~100 in the exp2 domain) underflows, and the epilogue sends its block to the running-max launch.
        float ls[2] = {0.0f, 0.0f};
        f32x16 negm;
        {
            float mx = -INFINITY;
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fmaxf(s[nb][0][r], s[nb][1][r]));
            mx = wave_pair_max(mx);
            const float m = mx > -INFINITY ? ceilf(mx) : 0.0f;
            negm = f32x16{} - m;
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                s[nb][0] -= m;
                s[nb][1] -= m;
            }
            ws_fence_negm(negm);
        }

        // P word w (0..15) of key block mb: (nb, kk, j) = (w / 8, 2 mb + (w / 4) % 2, w % 4); three stages
        float e0, e1, es;
        u32x4 grp;   // the 4-word group being packed (words w & ~3 .. w | 3)
        auto stage_e = [&](int mb, int w) __attribute__((always_inline)) {
            const int nb = w >> 3, r = 8 * ((w >> 2) & 1) + 2 * (w & 3);
            e0 = __builtin_amdgcn_exp2f(s[nb][mb][r]);
            e1 = __builtin_amdgcn_exp2f(s[nb][mb][r + 1]);
            asm volatile("" ::"v"(e0), "v"(e1));
        };
        auto stage_c = [&](int t, int mb, int w) __attribute__((always_inline)) {
            grp[w & 3] = pack_bf16x2(e0, e1);
            es = e0 + e1;
            asm volatile("" ::"v"(es));
            if ((w & 3) == 3) {   // the group is whole: P operand (nb, kk) of tile t
                *(lds_u32x4w*)(uintptr_t)p_addr(t, w >> 3, 2 * mb + ((w >> 2) & 1)) = grp;
            }
        };
        auto stage_d = [&](int w) __attribute__((always_inline)) {
            ls[w >> 3] += es;
            asm volatile("" ::"v"(ls[w >> 3]));
        };
        // P(0) of key block 0, serially
#pragma unroll
        for (int w = 0; w < 16; ++w) {
            stage_e(0, w);
            stage_c(0, 0, w);
            stage_d(w);
        }
        LR_WAIT_LGKM0();               // this wave's P writes are done
        LR_WAIT_VMCNT(WS_LOADS);       // K(1) has landed (K(2) may be in flight)
        block_barrier();               // P2: K(1) in every share; every A wave is done with K slot 0

        bf16x8 fr[4];
        fr[0] = kfrag(kslot(1), 0, 0);
        fr[1] = kfrag(kslot(1), 0, 1);
        fr[2] = kfrag(kslot(1), 0, 2);
        // The word stages of a group of 16 words (tile T, key block mb): slot sl runs D of word sl - 2, C of word
        // sl - 1, E of word sl, in that order (D reads the pair sum C is about to overwrite, C the exps E is about to
        // overwrite). Slots 0 and 1 finish the previous group's words 14 and 15.
        auto group_slot = [&](int sl, int pt, int pmb, bool prev, int ct, int cmb) __attribute__((always_inline)) {
            if (sl >= 2) stage_d(sl - 2);
            else if (prev) stage_d(14 + sl);
            if (sl >= 1) stage_c(ct, cmb, sl - 1);
            else if (prev) stage_c(pt, pmb, 15);
            stage_e(cmb, sl);
        };
        for (int t = 0; t < ntiles; ++t) {
            asm volatile("" : "+v"(lane_k));   // the fragment addresses are recomputed per step, not held
            const uint32_t kt = kslot(t + 1);
            if (needs_mask(t) && t > 0) {   // key block 0 of S(t) was masked in step t-1
                ws_fence_s(s);
                mask_block(t, 1);
            }
            __builtin_amdgcn_sched_barrier(0);
            // G0: S(t+1) key block 0 | P(t) key block 1 (after P(t) key block 0's last words, from step t-1's G1)
#pragma unroll
            for (int sl = 0; sl < 16; ++sl) {
                const int f = sl >> 1, nb = sl & 1;
                if (nb == 0 && f + 3 < 16) fr[(f + 3) & 3] = kfrag(kt, (f + 3) >> 3, (f + 3) & 7);
                if (f == 0) ws_qk_c(s[nb][0], fr[0], q[nb][0], negm);
                else ws_qk(s[nb][0], fr[f & 3], q[nb][f]);
                group_slot(sl, t, 0, t > 0, t, 1);
                if ((sl & 3) == 1) load_tile(t + WS_KNS, sl >> 2);
                __builtin_amdgcn_sched_barrier(0);
            }
            block_barrier();   // mid: B holds P(t-1), whose buffer G1 refills with P(t+1) key block 0
            if (needs_mask(t + 1)) {
                ws_fence_s(s);
                mask_block(t + 1, 0);
            }
            ws_fence_s0(s);   // G1's first exps read S(t+1) key block 0, which G0's last MFMAs wrote
            __builtin_amdgcn_sched_barrier(0);
            // G1: S(t+1) key block 1 | P(t+1) key block 0 (after P(t) key block 1's last words)
#pragma unroll
            for (int sl = 0; sl < 16; ++sl) {
                const int f = 8 + (sl >> 1), nb = sl & 1;
                if (nb == 0 && f + 3 < 16) fr[(f + 3) & 3] = kfrag(kt, (f + 3) >> 3, (f + 3) & 7);
                if (f == 8) ws_qk_c(s[nb][1], fr[f & 3], q[nb][0], negm);
                else ws_qk(s[nb][1], fr[f & 3], q[nb][f - 8]);
                group_slot(sl, t, 1, true, t + 1, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
            LR_WAIT_VMCNT(WS_LOADS);   // K(t+2) has landed in this wave's share (K(t+3) may be in flight)
            LR_WAIT_LGKM0();           // P writes done before B reads them
            block_barrier();           // end of step t
            const uint32_t kn = kslot(t + 2);
            fr[0] = kfrag(kn, 0, 0);
            fr[1] = kfrag(kn, 0, 1);
            fr[2] = kfrag(kn, 0, 2);
        }
        // the row sums, after the pending stages of the last group (P(ntiles): masked, zeros), to the pair's B wave
        stage_d(14);
        stage_c(ntiles, 0, 15);
        stage_d(15);
        LR_WAIT_VMCNT(0);
        const float l0 = wave_pair_sum(ls[0]), l1 = wave_pair_sum(ls[1]);
        typedef __attribute__((address_space(3))) float lds_f32;
        const uint32_t lbuf = pb_lds + (uint32_t)((ntiles & 1) * WS_PBUF);   // P buffer B no longer reads
        *(lds_f32*)(uintptr_t)(lbuf + lane * 4) = l0;
        *(lds_f32*)(uintptr_t)(lbuf + 256 + lane * 4) = l1;
        LR_WAIT_LGKM0();
        block_barrier();   // E1: row sums visible (B runs its last PV meanwhile)
    } else {
        // ================================================================ wave B: PV
        f32x16 o[2][4];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
            for (int db = 0; db < 4; ++db) o[nb][db] = f32x16{};
        block_barrier();   // P1
        block_barrier();   // P2
        bf16x8 fr[4];
        u32x4 pv[2][4];
        auto pv_step = [&](int t, bool mid) __attribute__((always_inline)) {
            // PV(t): O += V(t)^T P(t); P operands from LDS; a mid barrier after the first half when mid is set
            const uint32_t vt = vslot(t);
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) pv[nb][kk] = *(lds_u32x4*)(uintptr_t)p_addr(t, nb, kk);
            fr[0] = vfrag(vt, 0);
            fr[1] = vfrag(vt, 1);
            fr[2] = vfrag(vt, 2);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int sl = 0; sl < 32; ++sl) {
                const int f = sl >> 1, nb = sl & 1;
                if (nb == 0 && f + 3 < 16) fr[(f + 3) & 3] = vfrag(vt, f + 3);
                ws_mfma(o[nb][f & 3], fr[f & 3], __builtin_bit_cast(bf16x8, pv[nb][f >> 2]));
                __builtin_amdgcn_sched_barrier(0);
                if (mid && sl == 15) {
                    // the P operands are in registers: A may refill the buffer (its key block 0 half)
                    LR_WAIT_LGKM0();
                    block_barrier();
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        };
        for (int t = 0; t < ntiles; ++t) {
            // V(t) into its slot (V(t-2)'s, read in step t-1)
#pragma unroll
            for (int j = 0; j < WS_LOADS; ++j) load_tile(t, j);
            if (t == 0) {
                block_barrier();   // mid
            } else {
                pv_step(t - 1, true);
            }
            LR_WAIT_VMCNT(0);   // V(t) has landed in this wave's share
            block_barrier();    // end of step t
        }
        pv_step(ntiles - 1, false);
        block_barrier();   // E1: A's row sums
        typedef __attribute__((address_space(3))) const float lds_f32c;
        const uint32_t lbuf = pb_lds + (uint32_t)((ntiles & 1) * WS_PBUF);
        const float lsum[2] = {*(lds_f32c*)(uintptr_t)(lbuf + lane * 4), *(lds_f32c*)(uintptr_t)(lbuf + 256 + lane * 4)};
        bool overflow = false;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            const int qrow = wrow0 + 32 * nb + n;
            const float l = lsum[nb];
            const float inv = 1.0f / l;
            bool bad = !__builtin_isfinite(l) || !(l >= 0x1p-60f);   // overflowed, or underflowed under the shared reference
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
    }
}

template <int QK>
hipError_t launch_ws_t(const AttnArgs& a, hipStream_t stream) {
    const int64_t nqb = (a.W + WS_BM - 1) / WS_BM;
    const int64_t blocks = nqb * a.H;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL((attn_ws_kernel<QK>), dim3((unsigned)blocks), dim3(2 * WS_PAIRS * 64), 0, stream, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_ws(const AttnArgs& a, int qk, hipStream_t stream) {
    if (a.causal) return hipErrorInvalidValue;
    switch (qk) {
        case TABLE_NONE: return launch_ws_t<TABLE_NONE>(a, stream);
        case TABLE_COSSIN_F32: return launch_ws_t<TABLE_COSSIN_F32>(a, stream);
        case TABLE_MAT2_BF16: return launch_ws_t<TABLE_MAT2_BF16>(a, stream);
        case TABLE_MAT2_F32: return launch_ws_t<TABLE_MAT2_F32>(a, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace lr
