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
//  * The default kernel (attn_fwd_pipe_kernel) keeps K and V tiles row-major in an LDS ring filled by direct
//    global->LDS loads and reads V transposed (ds_read_b64_tr_b16); the QK^T MFMAs of the next tile run interleaved
//    with the softmax VALU work of the current one. Variants: 4-wave blocks (two per CU), 64 queries per wave, a
//    ping-pong pair of wave groups, and the first register-staged kernel (V^T formed by a register transpose).
//  * Workgroups are remapped so that each XCD works on whole heads (its own L2 holds that head's K/V).
//  * FUSEQ: the query block's per-head RMSNorm and RoPE are applied in registers before the first MFMA.
#include "lr_common.h"
#include "lr_kernels.h"

namespace lr {

namespace {

#include "attn_common.inc"

// The register-staged kernel: K/V tiles pass through VGPRs into a 2-stage LDS ring, V^T is formed by a register
// transpose. Kept as the reference point for the pipelined kernel below.
template <int QW, int NW, bool FUSEQ>
__global__ __launch_bounds__(NW * 64, 1) void attn_fwd_regstage_kernel(AttnArgs a) {
    constexpr int NQB = QW / 32;  // 32-query blocks per wave
    constexpr int BM = QW * NW;   // queries per workgroup
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    __shared__ __attribute__((aligned(16))) uint16_t Ks[2][BN * D];
    __shared__ __attribute__((aligned(16))) uint16_t Vs[2][D * BN];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 31, hf = lane >> 5;

    // XCD-aware mapping: hardware workgroup b runs on XCD b % 8; give each XCD a contiguous range of logical ids
    // (consecutive query blocks of the same head) so its L2 serves one head's K/V to all its CUs.
    const int nwg = gridDim.x, b = blockIdx.x;
    const int per = nwg >> 3, rem = nwg & 7, xcd = b & 7, idx = b >> 3;
    const int logical = xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
    const int nqb = (a.W + BM - 1) / BM;
    const int head = logical / nqb, qblk = logical - head * nqb;
    const int hk = head / a.G;
    const int row0 = qblk * BM, wrow0 = row0 + wave * QW;
    const int last_row = min(row0 + BM, a.W) - 1;
    int ntiles = (a.nkeys + BN - 1) / BN;
    if (a.causal) ntiles = min(ntiles, (a.p0 + last_row) / BN + 1);
    const uint16_t* kbase = a.k + (int64_t)hk * a.k_hs;
    const uint16_t* vbase = a.v + (int64_t)hk * a.v_hs;

    // ---- staging roles: with 4 waves every thread moves 4 K chunks and one V unit; with 8, waves 0-3 move K and
    // waves 4-7 move V.
    constexpr bool SPLIT = NW == 8;
    const int st = SPLIT ? (tid & 255) : tid;           // staging thread index 0..255
    const bool do_k = !SPLIT || wave < 4, do_v = !SPLIT || wave >= 4;
    const int vc = st & 15, vkg = st >> 4;             // V unit: dims 8*vc..+8 of keys 4*vkg..+4
    u32x4 kreg[4], vreg[4];
    uint32_t kvalid = 0, vvalid = 0;   // per-chunk "key < nkeys" bits of a partial tile, applied at store time

    auto stage_load = [&](int t) {
        const int key0 = t * BN;
        const bool partial = key0 + BN > a.nkeys;
        if (do_k) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int u = st + 256 * i, r = u >> 4, c = u & 15;
                const int key = partial ? min(key0 + r, a.nkeys - 1) : key0 + r;
                kreg[i] = *reinterpret_cast<const u32x4*>(kbase + (int64_t)key * a.k_rs + 8 * c);
            }
            kvalid = 0;
            if (partial) {
#pragma unroll
                for (int i = 0; i < 4; ++i) kvalid |= (key0 + ((st + 256 * i) >> 4) < a.nkeys) ? (1u << i) : 0u;
            }
        }
        if (do_v) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = partial ? min(key0 + 4 * vkg + i, a.nkeys - 1) : key0 + 4 * vkg + i;
                vreg[i] = *reinterpret_cast<const u32x4*>(vbase + (int64_t)key * a.v_rs + 8 * vc);
            }
            vvalid = 0;
            if (partial) {
#pragma unroll
                for (int i = 0; i < 4; ++i) vvalid |= (key0 + 4 * vkg + i < a.nkeys) ? (1u << i) : 0u;
            }
        }
        return partial;
    };
    auto stage_store = [&](int buf, bool partial) {
        if (partial) {   // zero the keys past nkeys (their rows were loaded clamped)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (do_k && !(kvalid >> i & 1)) kreg[i] = u32x4{0, 0, 0, 0};
                if (do_v && !(vvalid >> i & 1)) vreg[i] = u32x4{0, 0, 0, 0};
            }
        }
        if (do_k) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int u = st + 256 * i, r = u >> 4, c = u & 15;
                *reinterpret_cast<u32x4*>(&Ks[buf][k_lds(r, c)]) = kreg[i];
            }
        }
        if (do_v) {
            // 4 keys x 8 dims -> 8 rows of V^T (4 keys each). Lanes with odd vc write the rows in the order e ^ 1
            // so that every store instruction spreads over both row parities (all 64 banks).
            const bool odd = vc & 1;
            const int cc = vkg >> 1, hh = vkg & 1;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                uint32_t lo[2], hi[2];
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    const int ee = e ^ s, w = ee >> 1;
                    if (ee & 1) {
                        lo[s] = (vreg[0][w] >> 16) | (vreg[1][w] & 0xffff0000u);
                        hi[s] = (vreg[2][w] >> 16) | (vreg[3][w] & 0xffff0000u);
                    } else {
                        lo[s] = (vreg[0][w] & 0xffffu) | (vreg[1][w] << 16);
                        hi[s] = (vreg[2][w] & 0xffffu) | (vreg[3][w] << 16);
                    }
                }
                const int ee = odd ? (e ^ 1) : e;
                const int d = 8 * vc + ee;
                const u32x2 val = odd ? u32x2{lo[1], hi[1]} : u32x2{lo[0], hi[0]};
                *reinterpret_cast<u32x2*>(&Vs[buf][v_lds(d, cc) + 4 * hh]) = val;
            }
        }
    };

    // ---- queries
    bf16x8 qf[NQB][8];
#pragma unroll
    for (int nb = 0; nb < NQB; ++nb) {
        if constexpr (FUSEQ)
            load_q_fused_any(a, wrow0 + 32 * nb + n, head, hf, qf[nb]);
        else
            load_q_plain(a, wrow0 + 32 * nb + n, head, hf, qf[nb]);
    }

    stage_store(0, stage_load(0));
    __syncthreads();

    f32x16 o[4][NQB];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int nb = 0; nb < NQB; ++nb) o[db][nb] = f32x16{};
    float m_used[NQB], l_sum[NQB];
#pragma unroll
    for (int nb = 0; nb < NQB; ++nb) {
        m_used[nb] = -INFINITY;
        l_sum[nb] = 0.0f;
    }

    const int pr = key_perm(n);          // K row (within a 32-key block) this lane's A operand reads
    const float c = a.c;

    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        const bool more = t + 1 < ntiles;
        bool next_partial = false;
        if (more) next_partial = stage_load(t + 1);

        // ---- S^T = K Q^T for 64 keys x QW queries
        f32x16 s[2][NQB];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int nb = 0; nb < NQB; ++nb) s[mb][nb] = f32x16{};
        const uint16_t* kt = Ks[buf];
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) {
                const bf16x8 kf = *reinterpret_cast<const bf16x8*>(kt + k_lds(32 * mb + pr, 2 * ks + hf));
#pragma unroll
                for (int nb = 0; nb < NQB; ++nb)
                    s[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[nb][ks], s[mb][nb], 0, 0, 0);
            }
        }

        // ---- mask (only tiles that reach past nkeys or, when causal, past some query's position)
        const int key0 = t * BN;
        const bool need_mask = key0 + BN > a.nkeys || (a.causal && key0 + BN - 1 > a.p0 + wrow0);
        if (need_mask) {
#pragma unroll
            for (int nb = 0; nb < NQB; ++nb) {
                const int pos = a.p0 + wrow0 + 32 * nb + n;
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int key = key0 + 32 * mb + 16 * (r >> 3) + 8 * hf + (r & 7);
                        const bool vis = key < a.nkeys && (!a.causal || key <= pos);
                        if (!vis) s[mb][nb][r] = -INFINITY;
                    }
            }
        }

        // ---- online softmax (exp2 domain), P -> bf16 B operands of the PV MFMAs
        bf16x8 pf[NQB][4];
#pragma unroll
        for (int nb = 0; nb < NQB; ++nb) {
            float mx = s[0][nb][0];
#pragma unroll
            for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[0][nb][r]);
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[1][nb][r]);
            mx = wave_pair_max(mx) * c;
            const bool raise = mx > m_used[nb] + RESCALE_TAU;
            if (__builtin_amdgcn_ballot_w64(raise)) {
                const float mn = fmaxf(m_used[nb], mx);
                // a row's first visible tile is tile 0 (key 0 is visible to every query), so m_used is finite after
                // it; the guard keeps a (never expected) -inf - -inf from turning into NaN
                const float alpha = m_used[nb] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_used[nb] - mn);
                l_sum[nb] *= alpha;
#pragma unroll
                for (int db = 0; db < 4; ++db) o[db][nb] *= alpha;
                m_used[nb] = mn;
            }
            const float nm = -m_used[nb];
            float ls = 0.0f;
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    bf16x8 f;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const float p = __builtin_amdgcn_exp2f(fmaf(s[mb][nb][8 * half + j], c, nm));
                        ls += p;
                        f[j] = (bf16)p;
                    }
                    pf[nb][2 * mb + half] = f;
                }
            }
            l_sum[nb] += ls;
        }

        // ---- O^T += V^T P^T
        const uint16_t* vt = Vs[buf];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const bf16x8 vf = *reinterpret_cast<const bf16x8*>(vt + v_lds(32 * db + n, 2 * kk + hf));
#pragma unroll
                for (int nb = 0; nb < NQB; ++nb)
                    o[db][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[nb][kk], o[db][nb], 0, 0, 0);
            }
        }

        if (more) stage_store(buf ^ 1, next_partial);
        __syncthreads();
    }

    // ---- epilogue: O / l -> bf16 rows
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
                for (int g = 0; g < 4; ++g) {
                    const f32x16& acc = o[db][nb];
                    u32x2 w;
                    w[0] = pack_bf16x2(acc[4 * g] * inv, acc[4 * g + 1] * inv);
                    w[1] = pack_bf16x2(acc[4 * g + 2] * inv, acc[4 * g + 3] * inv);
                    *reinterpret_cast<u32x2*>(dst + 32 * db + 8 * g) = w;
                }
        }
    }
}

// ------------------------------------------------------------------------------------------------ pipelined kernel
// K and V tiles both live row-major in LDS ([64 keys][128 dims], 16 KB each) in a 3-stage ring, filled by direct
// global->LDS loads (global_load_lds_dwordx4: no VGPRs, no VALU). V is read transposed for the PV operand with
// ds_read_b64_tr_b16. Per tile t a wave runs
//   A: S(t+1) = K(t+1) Q^T on MFMA, interleaved with the softmax of S(t) on VALU (independent registers);
//   B: O += V(t)^T P(t);
//   the direct loads of K(t+3) and V(t+2), a wait for K(t+2) and V(t+1), one s_barrier.
// so the QK^T MFMAs of the next tile hide the exp/max/sum work of the current one, and every load has two tiles of
// compute to land.

// NW waves of NQB x 32 queries each; tiles of BT keys in an NS-stage K/V ring. NQB = 2 reads every K and V operand
// fragment from LDS once for two 32-query MFMAs, halving LDS traffic per MFMA, at one wave per SIMD (its registers
// need it); BT = 32 then keeps the two score buffers at 32 registers each.
// QK: how queries arrive -- QK_PLAIN (already normalised and rotated), a TableKind (RMSNorm + RoPE in registers
// with that table kind, its loads specialised), or QK_ANY (the table kind read at run time).
// VT: values arrive packed as V^T tiles ([128 dims][64 keys], 16 KB contiguous per tile, zero past nkeys), stored in
// LDS with 16-byte chunk c of dim row d at c ^ ((d >> 1) & 7), and the PV A operand is one ds_read_b128 per MFMA.
// REDO: the second launch after the 64-query-per-wave kernel (attn_pair.hip), same 256-query blocks: a workgroup
// recomputes its block only if that kernel marked one of the block's 64-row quarters (a NaN in its first row: some
// P overflowed its fixed reference), and exits otherwise.
template <int NW, int NQB, int BT, int NS, int QK, bool VT, bool REDO = false>
__global__ __launch_bounds__(NW * 64, NQB == 1 ? 8 / NW : 1)
__attribute__((amdgpu_waves_per_eu(NQB == 1 ? 2 : 1, NQB == 1 ? 2 : 1))) void attn_fwd_pipe_kernel(AttnArgs a) {
    static_assert(NS >= 2 && NS <= 4, "2- to 4-stage ring");
    static_assert(!VT || (BT == 64 && NQB == 1), "packed V^T tiles are 64 keys wide");
    // FOLD (fused queries on the scheduled 64-key shape): queries arrive multiplied by scale * log2(e), and the running
    // max m is subtracted by the score MFMAs themselves (their accumulator starts at -m instead of 0), so a score
    // register already holds s * scale * log2(e) - m and P = exp2(score) needs no per-score FMA.
    constexpr bool FOLD = QK != QK_PLAIN && NQB == 1 && BT == 64;
    static_assert(NQB == 1 || NQB == 2, "one or two 32-query blocks per wave");
    static_assert(BT == 32 || BT == 64, "32- or 64-key tiles");
    constexpr int BM = 32 * NQB * NW;
    constexpr int MB = BT / 32;        // 32-key score blocks per tile
    constexpr int KK = BT / 16;        // 16-key PV steps per tile
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
    const int nsplit = REDO ? 1 : (a.nsplit > 1 ? a.nsplit : 1);
    const int split = logical % nsplit, lq = logical / nsplit;
    const int head = lq / nqb, qblk = lq - head * nqb;
    if (nsplit > 1) {
        const int all_tiles = (a.nkeys + BT - 1) / BT;
        const int per_split = (all_tiles + nsplit - 1) / nsplit;
        const int key0 = split * per_split * BT;
        const int64_t t0 = (int64_t)split * per_split;
        a.k += t0 * BT * a.k_rs;
        a.v += VT ? t0 * TILE : t0 * BT * a.v_rs;
        a.nkeys = max(0, min(a.nkeys - key0, per_split * BT));
    }
    const int hk = head / a.G;
    const int row0 = qblk * BM, wrow0 = row0 + wave * 32 * NQB;
    const int last_row = min(row0 + BM, a.W) - 1;
    if constexpr (REDO) {
        static_assert(BM == 256, "the marked blocks are 256 queries");
        bool marked = false;
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            const int r = row0 + 64 * qq;
            if (r < a.W) marked = marked || (a.out[(int64_t)r * a.o_rs + head * D] & 0x7fffu) > 0x7f80u;
        }
        if (!marked) return;   // uniform over the workgroup: every thread read the same four values
    }
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
    const int64_t kstep = (int64_t)BT * a.k_rs, vstep = VT ? (int64_t)TILE : (int64_t)BT * a.v_rs;
    const uint16_t* kp[LOADS];
    const uint16_t* vp[LOADS];
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
        kp[j] = kbase + (int64_t)krow[j] * a.k_rs + kcol[j];
        if constexpr (VT) {
            // instruction j fills V^T dim rows 8i .. 8i+7 (i = wave + NW j): lane -> row 8i + (lane >> 3), LDS chunk
            // lane & 7, which holds logical chunk (lane & 7) ^ ((row >> 1) & 7)
            const int d = 8 * (wave + NW * j) + (lane >> 3);
            vp[j] = vbase + d * BT + 8 * ((lane & 7) ^ ((d >> 1) & 7));
        } else {
            vp[j] = vbase + (int64_t)krow[j] * a.v_rs + vcol;
        }
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
        if (VT || key0 + BT <= a.nkeys) {   // packed V^T tiles are whole (zero past nkeys)
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
    for (int nb = 0; nb < NQB; ++nb) {
        if constexpr (QK == QK_PLAIN)
            load_q_plain(a, wrow0 + 32 * nb + n, head, hf, qf[nb]);
        else if constexpr (QK == QK_ANY)
            load_q_fused_any(a, wrow0 + 32 * nb + n, head, hf, qf[nb]);
        else
            load_q_fused<QK>(a, wrow0 + 32 * nb + n, head, hf, qf[nb], FOLD ? a.c : 1.0f);
    }

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
    // packed V^T operand: lane reads dim row 32db + n, keys 16kk + 8hf .. +8 (logical chunk 2kk + hf)
    int vto[KK];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) vto[kk] = n * BT + 8 * ((2 * kk + hf) ^ ((n >> 1) & 7));

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
    // FOLD: m_used is also the offset the score MFMAs subtract; it starts at 0 (S(0) above was computed that way) and
    // `m_set` marks lanes whose reference has been taken from a finite tile max.
    float m_used[NQB], l_sum[NQB];
    bool m_set[NQB];
#pragma unroll
    for (int nb = 0; nb < NQB; ++nb) {
        m_used[nb] = FOLD ? 0.0f : -1e30f;
        l_sum[nb] = 0.0f;
        m_set[nb] = false;
    }
    f32x16 negm = f32x16{};   // FOLD: -m_used in every accumulator slot (the score MFMAs' initial accumulator)
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
            mx[nb] = FOLD ? wave_pair_max(m) : wave_pair_max(m) * c;
        }
    };
    // raise the running max (and rescale O, l) when a tile's max exceeds it by more than 2^8. FOLD: mx is relative to
    // the current offset, and the tile's scores sc (computed with the old offset) are shifted with it.
    auto rescale_for = [&](const float (&mx)[NQB], f32x16 (&sc)[NQB][MB]) {
#pragma unroll
        for (int nb = 0; nb < NQB; ++nb) {
            if constexpr (FOLD) {
                const bool want = (!m_set[nb] && mx[nb] > -INFINITY) || mx[nb] > RESCALE_TAU;
                if (__builtin_amdgcn_ballot_w64(want)) {
                    const float d = want ? mx[nb] : 0.0f;
                    const float alpha = m_set[nb] ? __builtin_amdgcn_exp2f(-d) : 1.0f;   // O, l are still 0 if unset
                    m_used[nb] += d;
                    m_set[nb] = m_set[nb] || want;
                    l_sum[nb] *= alpha;
#pragma unroll
                    for (int db = 0; db < 4; ++db) o[nb][db] *= alpha;
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb) sc[nb][mb] -= d;
                    negm = f32x16{} - m_used[nb];
                }
            } else if (__builtin_amdgcn_ballot_w64(mx[nb] > m_used[nb] + RESCALE_TAU)) {
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
        if constexpr (NQB == 1 && BT == 64) {
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
                if constexpr (VT) {
                    return *reinterpret_cast<const bf16x8*>(vt + vto[kk] + 32 * BT * db);
                } else {
                    const uint16_t* p0 = vt + vtr[db] + (16 * kk) * D;
                    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p0);
                    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p0 + 4 * D));
                    return __builtin_shufflevector(__builtin_bit_cast(bf16x4, lo), __builtin_bit_cast(bf16x4, hi), 0,
                                                   1, 2, 3, 4, 5, 6, 7);
                }
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
                        fr[s & 3], qf[0][s >> 1], s < 2 ? (FOLD ? negm : f32x16{}) : sn[0][s & 1], 0, 0, 0);
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
                    const float e0 = FOLD ? sc[0][kk >> 1][r] : fmaf(sc[0][kk >> 1][r], c, nm);
                    const float e1 = FOLD ? sc[0][kk >> 1][r + 1] : fmaf(sc[0][kk >> 1][r + 1], c, nm);
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
            mx[0] = FOLD ? wave_pair_max(mloc) : wave_pair_max(mloc) * c;
            if (t + 1 < ntiles && !needs_mask(t + 1)) rescale_for(mx, sn);
            // K(t+2) and V(t+1) must have landed; the loads of the last NS-2 steps (all refills while this step
            // refilled) may stay in flight
            if (NS == 2 || !refilled) LR_WAIT_VMCNT(0);
            else LR_WAIT_VMCNT((NS - 2) * 2 * LOADS);
            block_barrier();
            return;
        }
        bf16x8 pf[NQB][KK];
        auto exps = [&]() {
#pragma unroll
            for (int nb = 0; nb < NQB; ++nb) {
                const float nm = -m_used[nb];
                float ls = l_sum[nb];
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        // scalars, not a u32x4 indexed in a loop: hipcc 7.2 folds __builtin_bit_cast(bf16x2, w[j])
                        // of a vector element to w[0] for every j
                        uint32_t w[4];
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            w[j] = pack_bf16x2(__builtin_amdgcn_exp2f(fmaf(sc[nb][mb][8 * hh + 2 * j], c, nm)),
                                               __builtin_amdgcn_exp2f(fmaf(sc[nb][mb][8 * hh + 2 * j + 1], c, nm)));
                        // the row sum of the bf16 P exactly as the PV MFMA consumes it
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            ls = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w[j]), ones2, ls, false);
                        pf[nb][2 * mb + hh] = __builtin_bit_cast(bf16x8, u32x4{w[0], w[1], w[2], w[3]});
                    }
                }
                l_sum[nb] = ls;
            }
        };
        {
            // the last tile computes a throw-away S from a stale slot rather than branching: A and B stay one block
            const uint16_t* kt = Kr + ((t + 1) % NS) * TILE;
#pragma unroll
            for (int nb = 0; nb < NQB; ++nb)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) sn[nb][mb] = f32x16{};
#pragma unroll
            for (int ks = 0; ks < 8; ++ks)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) qk_block(kt, ks, mb, sn);
            exps();
            // interleave: two K reads ahead, then 8 MB x (NQB x (1 MFMA, 6 VALU), 1 DS read)
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
            for (int i = 0; i < 8 * MB; ++i) {
#pragma unroll
                for (int nb = 0; nb < NQB; ++nb) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
        }
        // ---- B: O^T += V^T P^T, with the next tile's max on the VALU
        const uint16_t* vt = Vr + (t % NS) * TILE;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                bf16x8 vf;
                if constexpr (VT) {
                    vf = *reinterpret_cast<const bf16x8*>(vt + vto[kk] + 32 * BT * db);
                } else {
                    const uint16_t* p0 = vt + vtr[db] + (16 * kk) * D;
                    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p0);
                    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p0 + 4 * D));
                    vf = __builtin_shufflevector(__builtin_bit_cast(bf16x4, lo), __builtin_bit_cast(bf16x4, hi), 0, 1,
                                                 2, 3, 4, 5, 6, 7);
                }
#pragma unroll
                for (int nb = 0; nb < NQB; ++nb)
                    o[nb][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[nb][kk], o[nb][db], 0, 0, 0);
            }
        }
        tile_max(sn, mx);
        if (t + 1 < ntiles && !needs_mask(t + 1)) rescale_for(mx, sn);
        // ---- K(t+2) and V(t+1) (issued a step ago with 3 stages, at this step's start with 2) must have landed
        if (NS == 2 || !refilled) LR_WAIT_VMCNT(0);
        else LR_WAIT_VMCNT((NS - 2) * 2 * LOADS);
        block_barrier();
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

// ------------------------------------------------------------------------------------------------ ping-pong kernel
// Eight waves in two groups of four (waves w and w + 4 share a SIMD). Each wave alternates two clusters per tile t:
//   M(t): S(t+1) = K(t+1) Q^T and O += V(t)^T P(t) -- MFMAs and their LDS operand reads only;
//   V(t): mask / max / rescale / exp2 / bf16 packing / row sums of S(t+1) -> P(t+1), and the direct loads of
//         K(t+4) and V(t+3) -- VALU and VMEM only.
// Group 1 trails group 0 by one cluster, and every cluster ends at a workgroup barrier, so while one wave of a SIMD
// issues back-to-back MFMAs the other runs its softmax on the VALU. K and V tiles sit in a 4-stage ring (128 KB):
// a slot is refilled two clusters after its last reader and read at least four clusters after the refill is issued.
constexpr int PP_STAGES = 4;

__device__ __forceinline__ void wait_vm_le(int n) {
    // s_waitcnt takes an immediate: the counts that occur here are 0, 2, 4, 6, 8
    if (n >= 8) LR_WAIT_VMCNT(8);
    else if (n >= 6) LR_WAIT_VMCNT(6);
    else if (n >= 4) LR_WAIT_VMCNT(4);
    else if (n >= 2) LR_WAIT_VMCNT(2);
    else LR_WAIT_VMCNT(0);
}

template <bool FUSEQ>
__global__ __launch_bounds__(512, 1) void attn_fwd_pp_kernel(AttnArgs a) {
    constexpr int NW = 8, BM = 32 * NW, TILE = BN * D, LOADS = 16 / NW;
    __shared__ __attribute__((aligned(1024))) uint16_t Kr[PP_STAGES * TILE];
    __shared__ __attribute__((aligned(1024))) uint16_t Vr[PP_STAGES * TILE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 31, hf = lane >> 5;
    const int grp = wave >> 2;

    const int nwg = gridDim.x, b = blockIdx.x;
    const int per = nwg >> 3, rem = nwg & 7, xcd = b & 7, idx = b >> 3;
    const int logical = xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
    const int nqb = (a.W + BM - 1) / BM;
    const int head = logical / nqb, qblk = logical - head * nqb;
    const int hk = head / a.G;
    const int row0 = qblk * BM, wrow0 = row0 + wave * 32;
    const int last_row = min(row0 + BM, a.W) - 1;
    int ntiles = (a.nkeys + BN - 1) / BN;
    if (a.causal) ntiles = min(ntiles, (a.p0 + last_row) / BN + 1);
    const uint16_t* kbase = a.k + (int64_t)hk * a.k_hs;
    const uint16_t* vbase = a.v + (int64_t)hk * a.v_hs;

    // ---- direct loads (as in the pipelined kernel)
    const int lrow = lane >> 4, lchunk = lane & 15;
    int krow[LOADS], kcol[LOADS];
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
        krow[j] = 4 * (wave + NW * j) + lrow;
        kcol[j] = 8 * (lchunk ^ (krow[j] & 15));
    }
    const int vcol = 8 * (lchunk ^ (lrow << 2));
    const uint32_t kr_lds = lds_addr(Kr), vr_lds = lds_addr(Vr);
    const int64_t kstep = (int64_t)BN * a.k_rs, vstep = (int64_t)BN * a.v_rs;
    const uint16_t* kp[LOADS];
    const uint16_t* vp[LOADS];
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
        kp[j] = kbase + (int64_t)krow[j] * a.k_rs + kcol[j];
        vp[j] = vbase + (int64_t)krow[j] * a.v_rs + vcol;
    }
    auto issue_k = [&](int t) {
        const int key0 = t * BN;
        const uint32_t dst = kr_lds + 2 * ((t % PP_STAGES) * TILE + wave * 512);
        if (key0 + BN <= a.nkeys) {
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
    auto issue_v = [&](int t) {
        const int key0 = t * BN;
        const uint32_t dst = vr_lds + 2 * ((t % PP_STAGES) * TILE + wave * 512);
        if (key0 + BN <= a.nkeys) {
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
    // loads issued by V(x): K(x+4) and V(x+3) while those tiles exist
    auto loads_in = [&](int x) { return (x + 4 < ntiles ? LOADS : 0) + (x + 3 < ntiles ? LOADS : 0); };

    // ---- queries
    bf16x8 qf[8];
    if constexpr (FUSEQ)
        load_q_fused_any(a, wrow0 + n, head, hf, qf);
    else
        load_q_plain(a, wrow0 + n, head, hf, qf);

    const int pr = key_perm(n);
    int kfrag[2];
    kfrag[0] = pr * D;
    kfrag[1] = (32 + pr) * D;
    const int kswz = pr & 15;
    const int g = lane >> 4, sl = lane & 15;
    int vtr[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) {
        const int chunk = 4 * (db ^ (sl >> 2)) + 2 * (g & 1) + ((sl & 3) >> 1);
        vtr[db] = (8 * (g >> 1) + (sl >> 2)) * D + 8 * chunk + 4 * (sl & 1);
    }
    typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;

    auto qk_block = [&](const uint16_t* kt, int ks, int mb, f32x16& acc) {
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(kt + kfrag[mb] + 8 * ((2 * ks + hf) ^ kswz));
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], acc, 0, 0, 0);
    };
    auto pv_block = [&](const uint16_t* vt, int kk, int db, const bf16x8& p, f32x16& acc) {
        const uint16_t* p0 = vt + vtr[db] + (16 * kk) * D;
        const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p0);
        const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p0 + 4 * D));
        const bf16x8 vf = __builtin_shufflevector(__builtin_bit_cast(bf16x4, lo), __builtin_bit_cast(bf16x4, hi), 0, 1,
                                                  2, 3, 4, 5, 6, 7);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, p, acc, 0, 0, 0);
    };

    // ---- prologue: K(0..3), V(0..2) resident; S(0) and P(0)
    issue_k(0);
    issue_v(0);
    if (ntiles > 1) { issue_k(1); issue_v(1); }
    if (ntiles > 2) { issue_k(2); issue_v(2); }
    if (ntiles > 3) issue_k(3);
    LR_WAIT_VMCNT(0);
    block_barrier();

    f32x16 s[2];
    s[0] = f32x16{};
    s[1] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) qk_block(Kr, ks, mb, s[mb]);

    f32x16 o[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] = f32x16{};
    float m_used = -1e30f, l_sum = 0.0f;   // finite start: every alpha is exp2 of a finite value or of -inf
    const float c = a.c;
    const int pos = a.p0 + wrow0 + n;
    const bf16x2 ones2 = {(bf16)1.0f, (bf16)1.0f};
    bf16x8 pf[4];

    // softmax of the score tile t held in s -> pf (P(t)), with the running max and row sum
    auto softmax_tile = [&](int t) {
        const int key0 = t * BN;
        if (key0 + BN > a.nkeys || (a.causal && key0 + BN - 1 > a.p0 + wrow0)) {
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = key0 + 32 * mb + 16 * (r >> 3) + 8 * hf + (r & 7);
                    if (!(key < a.nkeys && (!a.causal || key <= pos))) s[mb][r] = -INFINITY;
                }
        }
        float mx = fmaxf(s[0][0], s[0][1]);
#pragma unroll
        for (int r = 2; r < 16; ++r) mx = fmaxf(mx, s[0][r]);
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[1][r]);
        mx = wave_pair_max(mx) * c;
        if (__builtin_amdgcn_ballot_w64(mx > m_used + RESCALE_TAU)) {
            const float mn = fmaxf(m_used, mx);
            const float alpha = __builtin_amdgcn_exp2f(m_used - mn);
            m_used = mn;
            l_sum *= alpha;
#pragma unroll
            for (int db = 0; db < 4; ++db) o[db] *= alpha;
        }
        const float nm = -m_used;
        float ls = l_sum;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                // scalars, not a u32x4 indexed in a loop: hipcc 7.2 folds __builtin_bit_cast(bf16x2, w[j]) of a
                // vector element to w[0] for every j
                uint32_t w[4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    w[j] = pack_bf16x2(__builtin_amdgcn_exp2f(fmaf(s[mb][8 * hh + 2 * j], c, nm)),
                                       __builtin_amdgcn_exp2f(fmaf(s[mb][8 * hh + 2 * j + 1], c, nm)));
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    ls = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w[j]), ones2, ls, false);
                pf[2 * mb + hh] = __builtin_bit_cast(bf16x8, u32x4{w[0], w[1], w[2], w[3]});
            }
        }
        l_sum = ls;
    };

    softmax_tile(0);
    block_barrier();                 // K slot 0 is free for K(4) once every wave has its S(0)
    if (grp == 1) block_barrier();   // group 1 trails by one cluster

    for (int t = 0; t < ntiles; ++t) {
        const bool has_next = t + 1 < ntiles;
        // ---- M(t)
        __builtin_amdgcn_s_setprio(1);
        {
            const uint16_t* vt = Vr + (t % PP_STAGES) * TILE;
            if (has_next) {
                const uint16_t* kt = Kr + ((t + 1) % PP_STAGES) * TILE;
                s[0] = f32x16{};
                s[1] = f32x16{};
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    qk_block(kt, i >> 1, i & 1, s[i & 1]);
                    pv_block(vt, i >> 2, i & 3, pf[i >> 2], o[i & 3]);
                }
                // operands: six reads ahead, then two MFMAs per three reads
                __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 16; ++i) pv_block(vt, i >> 2, i & 3, pf[i >> 2], o[i & 3]);
            }
        }
        __builtin_amdgcn_s_setprio(0);
        wait_vm_le(t >= 1 ? loads_in(t - 1) : 0);
        block_barrier();
        // ---- V(t)
        if (has_next) softmax_tile(t + 1);
        if (t + 4 < ntiles) issue_k(t + 4);
        if (t + 3 < ntiles) issue_v(t + 3);
        wait_vm_le((t >= 1 ? loads_in(t - 1) : 0) + loads_in(t));
        block_barrier();
    }
    if (grp == 0) block_barrier();   // group 0 leads by one cluster

    // ---- epilogue: O / l -> bf16 rows
    const int qrow = wrow0 + n;
    const float l = wave_pair_sum(l_sum);
    const float inv = 1.0f / l;
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

template <bool FUSEQ>
hipError_t launch_pp(const AttnArgs& a, hipStream_t stream) {
    const int64_t nqb = (a.W + 255) / 256;
    const int64_t blocks = nqb * a.H;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL((attn_fwd_pp_kernel<FUSEQ>), dim3((unsigned)blocks), dim3(512), 0, stream, a);
    return hipGetLastError();
}

template <int QW, int NW, bool FUSEQ>
hipError_t launch_regstage(const AttnArgs& a, hipStream_t stream) {
    constexpr int BM = QW * NW;
    const int64_t nqb = (a.W + BM - 1) / BM;
    const int64_t blocks = nqb * a.H;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL((attn_fwd_regstage_kernel<QW, NW, FUSEQ>), dim3((unsigned)blocks), dim3(NW * 64), 0, stream, a);
    return hipGetLastError();
}

template <int NW, int NQB, int BT, int NS, int QK, bool VT = false, bool REDO = false>
hipError_t launch_pipe(const AttnArgs& a, hipStream_t stream) {
    constexpr int BM = 32 * NQB * NW;
    const int64_t nqb = (a.W + BM - 1) / BM;
    const int64_t blocks = nqb * a.H * (!REDO && a.nsplit > 1 ? a.nsplit : 1);
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL((attn_fwd_pipe_kernel<NW, NQB, BT, NS, QK, VT, REDO>), dim3((unsigned)blocks), dim3(NW * 64), 0,
                       stream, a);
    return hipGetLastError();
}

// The 64-query-per-wave kernel, then the running-max kernel on the blocks it marked.
template <int QK, bool VT>
hipError_t launch_pair_checked(const AttnArgs& a, hipStream_t stream) {
    const hipError_t e = launch_pair(a, QK, VT, stream);
    if (e != hipSuccess) return e;
    return launch_pipe<8, 1, 64, VT ? 4 : 3, QK, VT, true>(a, stream);
}

// The warp-specialised kernel, then the running-max kernel on the blocks it marked (the same 256-query blocks).
template <int QK>
hipError_t launch_ws_checked(const AttnArgs& a, hipStream_t stream) {
    if (a.causal) return launch_pair_checked<QK, true>(a, stream);   // the warp-specialised kernel is non-causal
    const hipError_t e = launch_ws(a, QK, stream);
    if (e != hipSuccess) return e;
    return launch_pipe<8, 1, 64, 4, QK, true, true>(a, stream);
}

}  // namespace

hipError_t launch_split_combine(const AttnArgs& a, hipStream_t stream) {
    const int64_t rows = (int64_t)a.H * a.W;
    hipLaunchKernelGGL(attn_split_combine_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

int attention_block_rows(int config) {
    switch (config) {
        case ATTN_CFG_PIPE_W4: return 128;
        default: return 256;
    }
}

bool attention_config_reads_vt(int config) {
    return config == ATTN_CFG_AUTO || config == ATTN_CFG_PIPE_W8 || config == ATTN_CFG_PIPE_W4 ||
           config == ATTN_CFG_PAIR_W4 || config == ATTN_CFG_WS_W8 || config == ATTN_CFG_PAIR_SK_W4;
}

// The prepared-keys path over packed V^T tiles, queries fused with table kind K (the 64-key pipelined shapes).
template <int K>
hipError_t launch_vt(const AttnArgs& a, int config, hipStream_t stream) {
    switch (config) {
        case ATTN_CFG_PIPE_W8: return launch_pipe<8, 1, 64, 4, K, true>(a, stream);
        case ATTN_CFG_PIPE_W4: return launch_pipe<4, 1, 64, 2, K, true>(a, stream);
        case ATTN_CFG_PAIR_W4:
        case ATTN_CFG_PAIR_SK_W4: return launch_pair_checked<K, true>(a, stream);   // stream-K when a.sk_part is set
        case ATTN_CFG_WS_W8: return launch_ws_checked<K>(a, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_attention(const AttnArgs& a, bool fuse_q, bool v_t, int config, hipStream_t stream) {
    // the library's choice: the 64-query-per-wave kernel where queries are fused and values are packed V^T tiles (the
    // joint-attention path; measured at least as fast at every BASELINE shape), the 32-query-per-wave pipelined kernel
    // for plain attention over value rows
    if (config == ATTN_CFG_AUTO) config = v_t ? ATTN_CFG_PAIR_W4 : ATTN_CFG_PIPE_W8;
    if (v_t) {
        if (!fuse_q) return hipErrorInvalidValue;
        switch (a.table_kind) {
            case TABLE_NONE: return launch_vt<TABLE_NONE>(a, config, stream);
            case TABLE_COSSIN_F32: return launch_vt<TABLE_COSSIN_F32>(a, config, stream);
            case TABLE_MAT2_BF16: return launch_vt<TABLE_MAT2_BF16>(a, config, stream);
            case TABLE_MAT2_F32: return launch_vt<TABLE_MAT2_F32>(a, config, stream);
            default: return hipErrorInvalidValue;
        }
    }
    // values as rows: the plain attention entry points, and the fused call's row-reading configurations
    switch (config) {
        case ATTN_CFG_PIPE_W8:
            if (fuse_q) return hipErrorInvalidValue;   // the fused call reaches this shape through packed V^T
            return launch_pipe<8, 1, 64, 3, QK_PLAIN>(a, stream);
        case ATTN_CFG_PIPE_W4:   // 64 KB of LDS so that two 4-wave blocks share a CU
            if (fuse_q) return hipErrorInvalidValue;
            return launch_pipe<4, 1, 64, 2, QK_PLAIN>(a, stream);
        case ATTN_CFG_PAIR_W4:
            if (fuse_q) return hipErrorInvalidValue;
            return launch_pair_checked<QK_PLAIN, false>(a, stream);
        case ATTN_CFG_WIDE_W4:
            return fuse_q ? launch_pipe<4, 2, 32, 4, QK_ANY>(a, stream) : launch_pipe<4, 2, 32, 4, QK_PLAIN>(a, stream);
        case ATTN_CFG_REGSTAGE_W8:
            return fuse_q ? launch_regstage<32, 8, true>(a, stream) : launch_regstage<32, 8, false>(a, stream);
        case ATTN_CFG_PINGPONG_W8:
            return fuse_q ? launch_pp<true>(a, stream) : launch_pp<false>(a, stream);
        default:
            return hipErrorInvalidValue;
    }
}

}  // namespace lr
