// Flash-style joint attention for gfx950 (CDNA4): bf16 in, fp32 MFMA accumulation and softmax, bf16 out.
//
// Semantics follow the reference's shipping kernel kernels/cuda/qwen_image/attention.cu:253-444 (pattn2_kernel) as
// launched by src/engines/qwen_image/ops_launch.zig:163-172: O_i = softmax_j(scale * <q_i, k_j>) v_j over keys
// j < nkeys (and j <= p0 + i when causal, attention.cu:304), query head h reading kv head h / (H / HK)
// (attention.cu:264-266), keys past nkeys zero-filled and masked (attention.cu:275-276), P rounded to bf16 for the
// PV product (attention.cu:418-424), output rounded to bf16 (attention.cu:432-443). The design is CDNA4's own:
//
//  * Scores are computed transposed, S^T = K Q^T, on v_mfma_f32_32x32x16_bf16 (M = 32 keys, N = 32 queries). In the
//    32x32 accumulator layout lane l owns query column l % 32 and 16 key rows, so a row max is 15 in-register maxes
//    plus one v_permlane32_swap with the partner lane l ^ 32; no LDS round trip, no 32-lane butterfly.
//  * The K rows of each 32-key block are read in an order with bits 2 and 3 of the row index swapped. With that
//    order, accumulator registers 0-7 / 8-15 of a score block are exactly the B operand (8 consecutive keys per lane
//    half) of the next MFMA, O^T += V^T P^T: P never leaves registers.
//  * Online softmax in the exp2 domain with scale*log2(e) folded into one FMA; the running max is only raised (and O
//    rescaled) when a tile's max exceeds it by more than 2^8, so the 64-register O rescale is rare after the first
//    tiles. Exact: every P and l use the same reference max, which cancels in O / l.
//  * The kernel (attn_fwd_pipe_kernel) keeps K and V tiles row-major in an LDS ring filled by direct global->LDS
//    loads and reads V transposed (ds_read_b64_tr_b16); the QK^T MFMAs of the next tile run interleaved with the
//    softmax VALU work of the current one. 8-wave blocks (256 queries, two waves per SIMD) or 4-wave blocks (two per
//    CU). The fused joint attention runs the streaming kernel of attn_stream.hip instead.
//  * Workgroups are remapped so that each XCD works on whole heads (its own L2 holds that head's K/V).
//  * FUSEQ: the query block's per-head RMSNorm and RoPE are applied in registers before the first MFMA.
#include "lr_common.h"
#include "lr_kernels.h"

namespace lr {

namespace {

#include "attn_common.inc"

// ------------------------------------------------------------------------------------------------ pipelined kernel
// K and V tiles both live row-major in LDS ([64 keys][128 dims], 16 KB each) in a 3-stage ring, filled by direct
// global->LDS loads (global_load_lds_dwordx4: no VGPRs, no VALU). V is read transposed for the PV operand with
// ds_read_b64_tr_b16. Per tile t a wave runs
//   A: S(t+1) = K(t+1) Q^T on MFMA, interleaved with the softmax of S(t) on VALU (independent registers);
//   B: O += V(t)^T P(t);
//   the direct loads of K(t+3) and V(t+2), a wait for K(t+2) and V(t+1), one s_barrier.
// so the QK^T MFMAs of the next tile hide the exp/max/sum work of the current one, and every load has two tiles of
// compute to land.

// NW waves of 32 queries each (two waves per SIMD at NW = 8); 64-key tiles in an NS-stage K/V ring.
template <int NW, int NS>
__global__ __launch_bounds__(NW * 64, 8 / NW) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_fwd_pipe_kernel(
    AttnArgs a) {
    static_assert(NS >= 2 && NS <= 4, "2- to 4-stage ring");
    constexpr int NQB = 1;             // 32-query blocks per wave
    constexpr int BT = 64;             // keys per tile
    constexpr int BM = 32 * NQB * NW;
    constexpr int MB = BT / 32;        // 32-key score blocks per tile
    constexpr int TILE = BT * D;       // elements per K or V tile
    constexpr int LOADS = BT / 4 / NW; // direct loads (1 KB = 4 rows each) per wave per K or V tile
    static_assert(LOADS >= 1, "every wave loads");
    typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;
    __shared__ __attribute__((aligned(1024))) uint16_t Kr[NS * TILE];
    __shared__ __attribute__((aligned(1024))) uint16_t Vr[NS * TILE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 31, hf = lane >> 5;

    const int nwg = gridDim.x, b = blockIdx.x;
    const int per = nwg >> 3, rem = nwg & 7, xcd = b & 7, idx = b >> 3;
    const int logical = xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
    const int nqb = (a.W + BM - 1) / BM;
    // key split: workgroup (query block, split) takes key tiles [split * per_split, ...) as if they were all the keys
    const int nsplit = a.nsplit > 1 ? a.nsplit : 1;
    const int split = logical % nsplit, lq = logical / nsplit;
    const int head = lq / nqb, qblk = lq - head * nqb;
    if (nsplit > 1) {
        const int all_tiles = (a.nkeys + BT - 1) / BT;
        const int per_split = (all_tiles + nsplit - 1) / nsplit;
        const int key0 = split * per_split * BT;
        const int64_t t0 = (int64_t)split * per_split;
        a.k += t0 * BT * a.k_rs;
        a.v += t0 * BT * a.v_rs;
        a.nkeys = max(0, min(a.nkeys - key0, per_split * BT));
    }
    const int hk = head / a.G;
    const int row0 = qblk * BM, wrow0 = row0 + wave * 32 * NQB;
    const int last_row = min(row0 + BM, a.W) - 1;
    int ntiles = (a.nkeys + BT - 1) / BT;
    if (a.causal) ntiles = min(ntiles, (a.p0 + last_row) / BT + 1);
    const uint16_t* kbase = a.k + (int64_t)hk * a.k_hs;
    const uint16_t* vbase = a.v + (int64_t)hk * a.v_hs;

    // ---- direct loads: instruction i (0 .. BT/4 - 1) of a tile fills rows 4i..4i+3; lane -> row 4i + (lane >> 4) and LDS
    // chunk (lane & 15), which must hold logical chunk (lane & 15) ^ swizzle(row). Rows past nkeys read the last
    // valid row instead (finite data; those keys are masked and their V rows meet P = 0).
    const int lrow = lane >> 4, lchunk = lane & 15;
    int krow[LOADS], kcol[LOADS];
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
        krow[j] = 4 * (wave + NW * j) + lrow;
        kcol[j] = 8 * (lchunk ^ (krow[j] & 15));
    }
    const int vcol = 8 * (lchunk ^ (lrow << 2));   // rows 4i + lrow: (r & 3) == lrow
    const uint32_t kr_lds = lds_addr(Kr), vr_lds = lds_addr(Vr);
    // Source pointers of the next K and V tiles to load, advanced one tile per issue; a tile reaching past nkeys
    // takes the clamped path instead.
    const int64_t kstep = (int64_t)BT * a.k_rs, vstep = (int64_t)BT * a.v_rs;
    const uint16_t* kp[LOADS];
    const uint16_t* vp[LOADS];
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
        kp[j] = kbase + (int64_t)krow[j] * a.k_rs + kcol[j];
        vp[j] = vbase + (int64_t)krow[j] * a.v_rs + vcol;
    }
    auto issue_k = [&](int t, int slot) {
        const int key0 = t * BT;
        const uint32_t dst = kr_lds + 2 * (slot * TILE + wave * 512);
        if (key0 + BT <= a.nkeys) {
#pragma unroll
            for (int j = 0; j < LOADS; ++j) dma16(kp[j], dst + 2 * NW * 512 * j);
        } else {
#pragma unroll
            for (int j = 0; j < LOADS; ++j) {
                const int key = min(key0 + krow[j], a.nkeys - 1);
                dma16(kbase + (int64_t)key * a.k_rs + kcol[j], dst + 2 * NW * 512 * j);
            }
        }
#pragma unroll
        for (int j = 0; j < LOADS; ++j) kp[j] += kstep;
    };
    auto issue_v = [&](int t, int slot) {
        const int key0 = t * BT;
        const uint32_t dst = vr_lds + 2 * (slot * TILE + wave * 512);
        if (key0 + BT <= a.nkeys) {
#pragma unroll
            for (int j = 0; j < LOADS; ++j) dma16(vp[j], dst + 2 * NW * 512 * j);
        } else {
#pragma unroll
            for (int j = 0; j < LOADS; ++j) {
                const int key = min(key0 + krow[j], a.nkeys - 1);
                dma16(vbase + (int64_t)key * a.v_rs + vcol, dst + 2 * NW * 512 * j);
            }
        }
#pragma unroll
        for (int j = 0; j < LOADS; ++j) vp[j] += vstep;
    };

    // ---- queries (B operands of S^T = K Q^T), one set per 32-query block
    // ---- prologue loads: K(0 .. NS-1) and V(0 .. NS-2) into the ring first, so that their latency overlaps the
    // query loads (the query's own waits, issued after, are conservative for the ring loads: older loads finish first)
    for (int i = 0; i < NS && i < ntiles; ++i) issue_k(i, i);
    for (int i = 0; i < NS - 1 && i < ntiles; ++i) issue_v(i, i);
    bf16x8 qf[NQB][8];
#pragma unroll
    for (int nb = 0; nb < NQB; ++nb) load_q_plain(a, wrow0 + 32 * nb + n, head, hf, qf[nb]);

    // ---- per-lane LDS offsets
    const int pr = key_perm(n);
    int kfrag[MB];                       // K A-operand row offsets of the 32-key blocks (chunk added per k-step)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) kfrag[mb] = (32 * mb + pr) * D;
    const int kswz = pr & 15;            // (32 + pr) & 15 == pr & 15
    // V^T operand by transposed reads: lane (group g = lane >> 4, s = lane & 15) addresses row 16kk + 8h + 4part +
    // (s >> 2), dims 32db + 16(g & 1) + 4(s & 3) .. +4, h = g >> 1.
    const int g = lane >> 4, sl = lane & 15;
    int vtr[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) {
        const int chunk = 4 * (db ^ (sl >> 2)) + 2 * (g & 1) + ((sl & 3) >> 1);
        vtr[db] = (8 * (g >> 1) + (sl >> 2)) * D + 8 * chunk + 4 * (sl & 1);
    }

    // one K operand fragment, used by every query block
    auto qk_block = [&](const uint16_t* kt, int ks, int mb, f32x16 (&acc)[NQB][MB]) {
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(kt + kfrag[mb] + 8 * ((2 * ks + hf) ^ kswz));
#pragma unroll
        for (int nb = 0; nb < NQB; ++nb)
            acc[nb][mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[nb][ks], acc[nb][mb], 0, 0, 0);
    };

    // ---- K(0 .. NS-1) and V(0 .. NS-2) resident; S(0)
    LR_WAIT_VMCNT(0);
    block_barrier();
    f32x16 sA[NQB][MB], sB[NQB][MB];
#pragma unroll
    for (int nb = 0; nb < NQB; ++nb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) sA[nb][mb] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) qk_block(Kr, ks, mb, sA);
    block_barrier();   // every wave is done with K slot 0 before step 0 refills it

    f32x16 o[NQB][4];
#pragma unroll
    for (int nb = 0; nb < NQB; ++nb)
#pragma unroll
        for (int db = 0; db < 4; ++db) o[nb][db] = f32x16{};
    // m_used starts at a finite -1e30 (not -inf): every alpha below is exp2 of a finite value or of -inf (= 0).
    float m_used[NQB], l_sum[NQB];
#pragma unroll
    for (int nb = 0; nb < NQB; ++nb) {
        m_used[nb] = -1e30f;
        l_sum[nb] = 0.0f;
    }
    const float c = a.c;
    const bf16x2 ones2 = {(bf16)1.0f, (bf16)1.0f};

    // keys past nkeys and (causal) past the query's position -> -inf; only tiles that reach either limit
    auto needs_mask = [&](int t) {
        const int key0 = t * BT;
        return key0 + BT > a.nkeys || (a.causal && key0 + BT - 1 > a.p0 + wrow0);
    };
    auto mask_tile = [&](int t, f32x16 (&sc)[NQB][MB]) {
        const int key0 = t * BT;
#pragma unroll
        for (int nb = 0; nb < NQB; ++nb) {
            const int pos = a.p0 + wrow0 + 32 * nb + n;
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = key0 + 32 * mb + 16 * (r >> 3) + 8 * hf + (r & 7);
                    if (!(key < a.nkeys && (!a.causal || key <= pos))) sc[nb][mb][r] = -INFINITY;
                }
        }
    };
    // a query's max over a score tile, scaled into the exp2 domain (both lanes of the query agree)
    auto tile_max = [&](const f32x16 (&sc)[NQB][MB], float (&mx)[NQB]) {
#pragma unroll
        for (int nb = 0; nb < NQB; ++nb) {
            float m = fmaxf(sc[nb][0][0], sc[nb][0][1]);
#pragma unroll
            for (int r = 2; r < 16; ++r) m = fmaxf(m, sc[nb][0][r]);
#pragma unroll
            for (int mb = 1; mb < MB; ++mb)
#pragma unroll
                for (int r = 0; r < 16; ++r) m = fmaxf(m, sc[nb][mb][r]);
            mx[nb] = wave_pair_max(m) * c;
        }
    };
    // raise the running max (and rescale O, l) when a tile's max exceeds it by more than 2^8
    auto rescale_for = [&](const float (&mx)[NQB], f32x16 (&)[NQB][MB]) {
#pragma unroll
        for (int nb = 0; nb < NQB; ++nb) {
            if (__builtin_amdgcn_ballot_w64(mx[nb] > m_used[nb] + RESCALE_TAU)) {
                const float mn = fmaxf(m_used[nb], mx[nb]);
                const float alpha = __builtin_amdgcn_exp2f(m_used[nb] - mn);
                m_used[nb] = mn;
                l_sum[nb] *= alpha;
#pragma unroll
                for (int db = 0; db < 4; ++db) o[nb][db] *= alpha;
            }
        }
    };
    float mx_cur[NQB];
    tile_max(sA, mx_cur);
    if (!needs_mask(0)) rescale_for(mx_cur, sA);

    // One tile t. On entry: sc = S(t), its max mx, and -- unless tile t needs masking -- the running max already
    // raised for it. Then
    //   mask (only tiles at nkeys or the causal diagonal; branch): -inf the hidden keys, recompute mx, raise;
    //   refill the ring for later tiles;
    //   A: S(t+1) on the MFMAs  ||  P(t) = exp2(S(t) c - m), its row sums and bf16 packing on the VALU;
    //   B: O += V(t)^T P(t)     ||  the max of S(t+1) on the VALU;
    //   raise the running max for tile t+1 (rare, branch), wait for the next tiles, barrier.
    // A and B form one basic block, so the scheduler can interleave across all of it.
    auto step = [&](int t, f32x16 (&sc)[NQB][MB], f32x16 (&sn)[NQB][MB], float (&mx)[NQB]) {
        if (needs_mask(t)) {
            mask_tile(t, sc);
            tile_max(sc, mx);
            rescale_for(mx, sc);
        }
        // ---- refill: K(t+NS) into the slot K(t) left, V(t+NS-1) into the slot V(t-1) left (both read last step)
        const bool refilled = t + NS < ntiles;
        if (refilled) issue_k(t + NS, t % NS);
        if (t + NS - 1 < ntiles) issue_v(t + NS - 1, (t + NS - 1) % NS);
        {
            // Explicit schedule of the tile's 32 MFMA slots (one wave's instruction stream; a sched_barrier closes
            // every slot, so the compiler keeps each slot's work in it):
            //   slots 0-15   S(t+1) = K(t+1) Q^T, the two 32-key accumulator chains alternating;
            //   slots 16-31  O += V(t)^T P(t), 16-key step kk = (s - 16) / 4, the four 32-dim chains alternating;
            //   LDS operand fragments read 3 slots ahead into a 4-entry ring (K fragments, then V fragments);
            //   exp2 pair k of P(t) (k = 4 kk + j) in slot floor(3k / 2): VALU work spread over slots 0-22, and P
            //   for step kk complete before its first PV slot;
            //   the max of S(t+1) in slots 24-31, long after its MFMAs retired.
            const uint16_t* kt = Kr + ((t + 1) % NS) * TILE;
            const uint16_t* vt = Vr + (t % NS) * TILE;
            auto frag = [&](int f) -> bf16x8 {
                if (f < 16) {
                    const int ks = f >> 1, mb = f & 1;
                    return *reinterpret_cast<const bf16x8*>(kt + kfrag[mb] + 8 * ((2 * ks + hf) ^ kswz));
                }
                const int i = f - 16, kk = i >> 2, db = i & 3;
                const uint16_t* p0 = vt + vtr[db] + (16 * kk) * D;
                const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p0);
                const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p0 + 4 * D));
                return __builtin_shufflevector(__builtin_bit_cast(bf16x4, lo), __builtin_bit_cast(bf16x4, hi), 0, 1, 2,
                                               3, 4, 5, 6, 7);
            };
            bf16x8 fr[4];
            fr[0] = frag(0);
            fr[1] = frag(1);
            fr[2] = frag(2);
            const float nm = -m_used[0];
            float ls = l_sum[0];
            float mloc = -INFINITY;
            // packed bf16 pairs of P(t), scalars (hipcc 7.2 folds __builtin_bit_cast(bf16x2, w[j]) of a vector
            // element to w[0] for every j)
            uint32_t pw[16];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s = 0; s < 32; ++s) {
                if (s + 3 < 32) fr[(s + 3) & 3] = frag(s + 3);
                if (s < 16) {
                    sn[0][s & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        fr[s & 3], qf[0][s >> 1], s < 2 ? f32x16{} : sn[0][s & 1], 0, 0, 0);
                } else {
                    const int kk = (s - 16) >> 2, db = (s - 16) & 3;
                    const bf16x8 pb = __builtin_bit_cast(bf16x8, u32x4{pw[4 * kk], pw[4 * kk + 1], pw[4 * kk + 2],
                                                                       pw[4 * kk + 3]});
                    o[0][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fr[s & 3], pb, o[0][db], 0, 0, 0);
                }
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    if ((3 * k) / 2 != s) continue;
                    const int kk = k >> 2, j = k & 3, r = 8 * (kk & 1) + 2 * j;
                    const float e0 = fmaf(sc[0][kk >> 1][r], c, nm);
                    const float e1 = fmaf(sc[0][kk >> 1][r + 1], c, nm);
                    pw[k] = pack_bf16x2(__builtin_amdgcn_exp2f(e0), __builtin_amdgcn_exp2f(e1));
                    // the row sum of the bf16 P exactly as the PV MFMA consumes it
                    ls = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pw[k]), ones2, ls, false);
                }
                if (s >= 24) {
                    const int g = 4 * (s - 24);
#pragma unroll
                    for (int u = 0; u < 4; ++u) mloc = fmaxf(mloc, sn[0][(g + u) >> 4][(g + u) & 15]);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            l_sum[0] = ls;
            mx[0] = wave_pair_max(mloc) * c;
            if (t + 1 < ntiles && !needs_mask(t + 1)) rescale_for(mx, sn);
            // K(t+2) and V(t+1) must have landed; the loads of the last NS-2 steps (all refills while this step
            // refilled) may stay in flight
            if (NS == 2 || !refilled) LR_WAIT_VMCNT(0);
            else LR_WAIT_VMCNT((NS - 2) * 2 * LOADS);
            block_barrier();
        }
    };

    int t = 0;
    for (; t + 1 < ntiles; t += 2) {
        step(t, sA, sB, mx_cur);
        step(t + 1, sB, sA, mx_cur);
    }
    if (t < ntiles) step(t, sA, sB, mx_cur);

    // ---- epilogue: O / l -> bf16 rows (or, with a key split, this range's partial result)
    if (nsplit > 1) {
#pragma unroll
        for (int nb = 0; nb < NQB; ++nb) {
            const int qrow = wrow0 + 32 * nb + n;
            const float l = wave_pair_sum(l_sum[nb]);
            if (qrow < a.W) {
                const int64_t slot = ((int64_t)head * a.W + qrow) * nsplit + split;
                float* po = a.part_o + slot * D + 4 * hf;
#pragma unroll
                for (int db = 0; db < 4; ++db)
#pragma unroll
                    for (int gg = 0; gg < 4; ++gg)
                        *reinterpret_cast<f32x4*>(po + 32 * db + 8 * gg) =
                            f32x4{o[nb][db][4 * gg], o[nb][db][4 * gg + 1], o[nb][db][4 * gg + 2],
                                  o[nb][db][4 * gg + 3]};
                if (hf == 0) {
                    // an empty key range (l = 0) contributes nothing whatever its reference
                    a.part_ml[2 * slot] = l > 0.0f ? m_used[nb] : -INFINITY;
                    a.part_ml[2 * slot + 1] = l;
                }
            }
        }
        return;
    }
#pragma unroll
    for (int nb = 0; nb < NQB; ++nb) {
        const int qrow = wrow0 + 32 * nb + n;
        const float l = wave_pair_sum(l_sum[nb]);
        const float inv = 1.0f / l;
        if (qrow < a.W) {
            uint16_t* dst = a.out + (int64_t)qrow * a.o_rs + head * D + 4 * hf;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int gg = 0; gg < 4; ++gg) {
                    u32x2 w;
                    w[0] = pack_bf16x2(o[nb][db][4 * gg] * inv, o[nb][db][4 * gg + 1] * inv);
                    w[1] = pack_bf16x2(o[nb][db][4 * gg + 2] * inv, o[nb][db][4 * gg + 3] * inv);
                    *reinterpret_cast<u32x2*>(dst + 32 * db + 8 * gg) = w;
                }
        }
    }
}

// One wave per (head, query row): O = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s, M = max_s m_s, two dims a lane.
__global__ void attn_split_combine_kernel(AttnArgs a) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= (int64_t)a.H * a.W) return;
    const int head = (int)(r / a.W), qrow = (int)(r - (int64_t)head * a.W);
    const int ns = a.nsplit;
    const float* ml = a.part_ml + r * ns * 2;
    float M = -INFINITY;
    for (int s = 0; s < ns; ++s) M = fmaxf(M, ml[2 * s]);
    float L = 0.0f, o0 = 0.0f, o1 = 0.0f;
    for (int s = 0; s < ns; ++s) {
        const float m = ml[2 * s];
        if (m == -INFINITY) continue;
        const float w = __builtin_amdgcn_exp2f(m - M);
        L = fmaf(w, ml[2 * s + 1], L);
        const float* po = a.part_o + (r * ns + s) * D + 2 * lane;
        o0 = fmaf(w, po[0], o0);
        o1 = fmaf(w, po[1], o1);
    }
    const float inv = 1.0f / L;
    *reinterpret_cast<uint32_t*>(a.out + (int64_t)qrow * a.o_rs + head * D + 2 * lane) = pack_bf16x2(o0 * inv, o1 * inv);
}

template <int NW, int NS>
hipError_t launch_pipe(const AttnArgs& a, hipStream_t stream) {
    constexpr int BM = 32 * NW;
    const int64_t nqb = (a.W + BM - 1) / BM;
    const int64_t blocks = nqb * a.H * (a.nsplit > 1 ? a.nsplit : 1);
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL((attn_fwd_pipe_kernel<NW, NS>), dim3((unsigned)blocks), dim3(NW * 64), 0, stream, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_split_combine(const AttnArgs& a, hipStream_t stream) {
    const int64_t rows = (int64_t)a.H * a.W;
    hipLaunchKernelGGL(attn_split_combine_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

// Plain attention over value rows (queries already normalised and rotated): the 8-wave (256-query blocks) or 4-wave
// (128-query blocks, two per CU) pipelined kernel.
hipError_t launch_attention(const AttnArgs& a, int config, hipStream_t stream) {
    switch (config) {
        case ATTN_CFG_AUTO:
        case ATTN_CFG_PIPE_W8: return launch_pipe<8, 3>(a, stream);
        case ATTN_CFG_PIPE_W4: return launch_pipe<4, 2>(a, stream);   // 64 KB of LDS: two per CU
        default: return hipErrorInvalidValue;
    }
}

}  // namespace lr
