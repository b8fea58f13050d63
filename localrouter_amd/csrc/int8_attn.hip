// The INT8 attention chain for gfx950: the prep (K anchor, V channel abs-max, Q/K rotation + quantisation, V
// quantisation into transposed tiles) and the attention kernel (int8 MFMA for Q K^T and P V).
//
// Reference semantics (jayleaton/localrouter, comfy-kitchen 0.2.35 vendored at kernels/cuda/minimax/kitchen/):
//   detect_k_anchor        quant_qk_int8.cu:461-596
//   Hadamard rotations     quant_qk_int8.cu:75-155 (convrot4, the sign words, five xor butterflies, 1/sqrt(128))
//   Q/K quantisation       quant_qk_int8.cu:245-247 (scale = absmax / 127 + 1e-7), float_utils.cuh:40-51 (rn, sat)
//   V quantisation         quant_v_int8.cu:64-140 (per channel, max(absmax / 127, 1e-12))
//   attention              qk_int_sv_i8_cuda.cuh:56-770 with attn_utils.cuh:610-695 (update_mdo_i32_u8): per key
//                          tile the row max m_t of the scores, P = exp2(s - m_t + 7.9943534) rounded to u8 (so the
//                          tile's largest P is 255), the row sum taken over the rounded P, O accumulated in fp32 with
//                          the tile's scale exp2(m_t - m_running)
//
// gfx950 mapping of the attention kernel (one workgroup = 512 threads = 8 waves x 32 queries, two waves per SIMD):
//   S^T = K Q^T with v_mfma_i32_32x32x32_i8: the A operand is 32 key rows read from LDS in the order key_perm, which
//   makes the 16 scores a lane holds per 32-key block the 16 consecutive keys 16*(lane/32) .. + 15 -- exactly the
//   B operand layout of the P V product, so P goes from registers into the next MFMA with no shuffle.
//   The MFMA is signed x signed, the reference's P is unsigned: P is stored as P ^ 0x80 (= P - 128) and the missing
//   128 * sum_j v_j is added back per tile by one v_mfma_f32_32x32x2_f32 per 32-dim block whose A operand is the
//   tile's precomputed int16 column sums and B operand 128 * tile_scale, accumulating straight into O.
//   K, V^T and the per-tile aux block stream through a 4-stage LDS ring with direct global->LDS loads.
//   The query blocks of a last partial round of the compute units (at most half of them) are cut into up to 4 key
//   ranges, one workgroup each, whose rows i8_split_combine_kernel merges (launch_attention).
#include <limits.h>

#include <algorithm>
#include <math.h>

#include <type_traits>

#include "lr_common.h"
#include "lr_int8.h"

namespace lr {
namespace i8 {

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

constexpr float S_U8_OFFSET = 7.9943534f;  // log2(255): the tile's largest P becomes 255 (attn_utils.cuh:41)

// ------------------------------------------------------------------------------------------------ direct loads
#define LR_I8_WAIT_VMCNT(n) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory")

// One 16-byte-per-lane direct load, global -> LDS: lane l reads 16 bytes at base + voff and they land at LDS byte
// address lds + 16 * l. base and lds are wave-uniform (SGPRs); only the 32-bit offset is per lane.
__device__ __forceinline__ void dma16(const void* base, uint32_t voff, uint32_t lds) {
    // readfirstlane returns a signed int: widen through uint32_t, or the low half would be sign-extended into the
    // high half of the address
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const uint64_t sb = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32) |
                        (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
    // M0 named as clobbered: the compiler keeps no value of its own in it across the statement (the pragmas only
    // silence clang's warning that M0 is a reserved register)
    _Pragma("clang diagnostic push") _Pragma("clang diagnostic ignored \"-Winline-asm\"")
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sb),
                 "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory", "m0");
    _Pragma("clang diagnostic pop")
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

// ------------------------------------------------------------------------------------------------ prep helpers
// Exchange with lane ^ M. M < 16: inside each row of 16 lanes by DPP (a register move across lanes, no LDS round
// trip): quad_perm [1,0,3,2] / [2,3,0,1] for M = 1 / 2, row_ror:8 for M = 8 (a rotation by 8 inside a 16-lane row is
// xor 8); for M = 4 the lanes with bit 2 clear take row_shl:4 (lane i + 4), the others row_shr:4 (lane i - 4). M = 16:
// inside each 32-lane half (ds_swizzle, and 0x1f, xor 16).
template <int CTRL>
__device__ __forceinline__ int dpp_mov(int x) {
    return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xf, 0xf, true);
}
// the DPP control of the single-move exchanges (M = 1, 2, 8)
template <int M>
constexpr int xor_dpp_ctrl() { return M == 1 ? 0xb1 : M == 2 ? 0x4e : 0x128; }
template <int M>
__device__ __forceinline__ int xor_lane_i(int x) {
    if constexpr (M == 1 || M == 2 || M == 8) {
        return dpp_mov<xor_dpp_ctrl<M>()>(x);
    } else if constexpr (M == 4) {
        const int up = dpp_mov<0x104>(x), dn = dpp_mov<0x114>(x);
        return (threadIdx.x & 4) ? dn : up;
    } else {
        return __builtin_amdgcn_ds_swizzle(x, 0x1f | (M << 10));
    }
}
template <int M>
__device__ __forceinline__ float xor_lane(float x) {
    return __int_as_float(xor_lane_i<M>(__float_as_int(x)));
}
template <int M>
__device__ __forceinline__ double xor_lane(double x) {
    const uint64_t b = (uint64_t)__double_as_longlong(x);
    const uint32_t lo = (uint32_t)xor_lane_i<M>((int)(uint32_t)b), hi = (uint32_t)xor_lane_i<M>((int)(uint32_t)(b >> 32));
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// max over each group of LPR lanes (one row of 8 * LPR channels, 8 per lane)
template <int LPR>
__device__ __forceinline__ float max_row(float x) {
    x = fmaxf(x, xor_lane<1>(x));
    x = fmaxf(x, xor_lane<2>(x));
    x = fmaxf(x, xor_lane<4>(x));
    if (LPR == 16) x = fmaxf(x, xor_lane<8>(x));
    return x;
}

// max over the wave
__device__ __forceinline__ float max64(float x) {
    x = max_row<16>(x);
    x = fmaxf(x, xor_lane<16>(x));
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Round to nearest even, saturate to [-128, 127]; NaN -> 0 (float_utils.cuh:40-51). v_cvt_i32_f32 itself turns NaN
// into 0 and saturates out-of-range values (infinities included) to the int32 range, so after the rounding one
// integer clamp remains (written as asm: the conversion of NaN or of an out-of-range value is undefined in C++).
__device__ __forceinline__ int rn_sat(float x) {
    int i;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(i) : "v"(rintf(x)));
    return min(max(i, -128), 127);
}

// The low bytes of four ints as one little-endian word (v_perm_b32: byte selector 0x0c is zero)
__device__ __forceinline__ uint32_t pack_lo_bytes(int b0, int b1, int b2, int b3) {
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)b1, (uint32_t)b0, 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)b3, (uint32_t)b2, 0x0c0c0400u);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// The reference rotates a 128-channel row held as 4 channels per lane of 32 lanes (quant_qk_int8.cu:75-155):
// [sign flip], H4 on the lane's 4 channels, [five butterflies over lane bits 1, 2, 4, 8, 16, then * 1/sqrt(128)];
// a 64-channel row (convrot64) as 4 channels per lane of 16 lanes: H4, four butterflies over lane bits 1 .. 8, * 1/4.
// Here a lane L of a group of 16 (8 at head dim 64) holds 8 channels, those of the reference's lanes r = 2L and
// 2L + 1: the sign flip and the H4 act on each 4-channel half, the butterfly over lane bit 1 pairs the two halves in
// registers, and those over lane bits 2 .. 16 (2 .. 8) are butterflies over L's bits 1 .. 8 (1 .. 4). Every value
// sees the same operations in the same order as in the reference, so the results are the same bits.
// A butterfly gives the lane with bit M clear x + o and the other o - x (o the partner's value). For M = 1, 2, 8 the
// partner is one DPP move away, so it is o + (+-x): this lane's value with its sign flipped where bit M is set (exactly
// o - x in IEEE arithmetic), and the partner's value read straight into the add (v_add_f32_dpp): two instructions a
// value. For M = 4 the two directions are separate shifts: x + (lane i + 4) and (lane i - 4) - x, each with the shifted
// operand read into the add / subtract, then one select.
template <int M>
__device__ __forceinline__ void butterfly8(float (&x)[8], int L) {
#pragma clang fp contract(off)
    const uint32_t sgn = (L & M) ? 0x80000000u : 0u;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        if constexpr (M == 4) {
            const float up = __int_as_float(dpp_mov<0x104>(__float_as_int(x[c])));
            const float dn = __int_as_float(dpp_mov<0x114>(__float_as_int(x[c])));
            x[c] = (L & M) ? dn - x[c] : x[c] + up;
        } else {
            const float o = __int_as_float(dpp_mov<xor_dpp_ctrl<M>()>(__float_as_int(x[c])));
            x[c] = o + __uint_as_float(__float_as_uint(x[c]) ^ sgn);
        }
    }
}

template <int ROT>
__device__ __forceinline__ void rotate8(float (&x)[8], int L) {
#pragma clang fp contract(off)
    if (ROT == 128) {
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const int r = 2 * L + g;
            const uint32_t w = r < 8 ? 0x1035997bu : r < 16 ? 0x8087f5eeu : r < 24 ? 0xee2e4e1au : 0x71132418u;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint32_t flip = ((w >> ((r & 7) * 4 + c)) & 1u) ^ 1u;
                x[4 * g + c] = __uint_as_float(__float_as_uint(x[4 * g + c]) ^ (flip << 31));
            }
        }
    }
#pragma unroll
    for (int g = 0; g < 2; ++g) {
        float* y = x + 4 * g;
        const float a0 = y[0] + y[1], a1 = y[0] - y[1], a2 = y[2] + y[3], a3 = y[2] - y[3];
        y[0] = (a0 + a2) * 0.5f;
        y[1] = (a1 + a3) * 0.5f;
        y[2] = (a0 - a2) * 0.5f;
        y[3] = (a1 - a3) * 0.5f;
    }
    if (ROT == 128 || ROT == 64) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {  // lane bit 1: reference lane 2L adds, lane 2L + 1 subtracts its own value
            const float e = x[c], o = x[4 + c];
            x[c] = e + o;
            x[4 + c] = e - o;
        }
        butterfly8<1>(x, L);
        butterfly8<2>(x, L);
        butterfly8<4>(x, L);
        if (ROT == 128) butterfly8<8>(x, L);
        const float norm = ROT == 128 ? 0.1767766952966369f : 0.25f;
#pragma unroll
        for (int c = 0; c < 8; ++c) x[c] *= norm;
    }
}

__device__ __forceinline__ void load8(const uint16_t* p, float (&x)[8]) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        x[2 * j] = lo_bf16(w[j]);
        x[2 * j + 1] = hi_bf16(w[j]);
    }
}

// 8 values * inv, rounded and saturated to int8, as two little-endian words
__device__ __forceinline__ u32x2 pack_s8x8(const float (&x)[8], float inv) {
#pragma clang fp contract(off)
    int q[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) q[c] = rn_sat(x[c] * inv);
    return u32x2{pack_lo_bytes(q[0], q[1], q[2], q[3]), pack_lo_bytes(q[4], q[5], q[6], q[7])};
}

// ------------------------------------------------------------------------------------------------ fused rmsRope
// Kitchen.rmsRope (kernels/cuda/minimax/kitchen/rms_rope.cu:37-230, as src/engines/minimax_h3/launch.zig:421-441
// launches it) of one row held by a group of 16 lanes, lane L holding channels 8 L .. 8 L + 7, for the prep of
// lr_int8_attention_prep_rope:
//   rrms = 1 / sqrt(sum(x^2) / 128 + eps) and x * rrms * w, in double, rounded to fp32 and then to bf16 (the
//   normalised value the reference rounds before the rotation, rms_rope.cu:143-150);
//   pairs (i, i + rot / 2), i < rot / 2, rotated by the table's [f00 f01; f10 f11] (rope_device.cuh:65-98) in fp32
//   and rounded to bf16 (the value the reference stores); channels >= rot keep the normalised value.
// The sum of squares of bf16 values is exact in double (for rows whose values span less than 2^30 in magnitude), sqrt
// and division are correctly rounded, the normalised values are those of the double computation (norm_bf16_exact),
// and the products in the rotation are products of bf16 values (exact in fp32), so each result is the same bits as
// the CPU restatement (oracle/lro.c, lro_rms_rope_ex with round_norm) rounded to bf16.
struct RopeTab {
    uint32_t w[8];  // this lane's row of each of its 8 pairs' matrices: (f00, f01) or (f10, f11), bf16
};

// The table entries of token `token` for lane L: pairs 8 pc .. 8 pc + 7 (pc = L or L - rot / 16), of each pair's
// [2][2] matrix the row this lane's output needs (row 0 for the first half's lanes, row 1 for the second's): eight
// 4-byte loads. (Lanes past the rotated channels load pair chunk 0 too, unused: no branch around the loads.)
__device__ __forceinline__ RopeTab rope_tab_load(const PrepArgs& a, int token, int L) {
    RopeTab t;
    const int hc = a.rope_rot >> 4;
    const int pc = L < hc ? L : (L < 2 * hc ? L - hc : 0);
    const uint16_t* src = a.rope_tab + (int64_t)token * a.tab_rs + 32 * pc + (L >= hc && L < 2 * hc ? 2 : 0);
#pragma unroll
    for (int j = 0; j < 8; ++j) t.w[j] = *reinterpret_cast<const uint32_t*>(src + 4 * j);
    return t;
}

// The table rows of a block's 64 rows staged in LDS, row r at byte 4 rot r (the table row's first 4 rot bytes:
// [rot/2 pairs][2][2] bf16), moved by direct global -> LDS loads: rot / 4 loads of 1 KB (64 lanes x 16 bytes), spread
// over the block's four waves and issued before the block's own row loads, so that one wait covers both. Rows
// row_of(r) never precede row_of(0) and lie within 64 rows of it: the per-lane byte offsets from row row_of(0) fit in
// 32 bits (tab_rs <= 2^24, checked by the caller).
__host__ __device__ constexpr int tab_lds_bytes(int rot) { return 64 * 4 * rot; }

// Issue the loads of table rows row_of(r), r < 64, into lds; the caller waits (vmcnt 0) and synchronises the block
// before reading them.
template <typename RowOf>
__device__ __forceinline__ void rope_tab_dma(const PrepArgs& a, uint8_t* lds, RowOf row_of) {
    const int nch = a.rope_rot >> 2;   // 16-byte chunks a row
    const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int r0 = row_of(0);
    const uint16_t* base = a.rope_tab + (int64_t)r0 * a.tab_rs;
    for (int i = wave; i < nch; i += 4) {   // load i: chunks 64 i .. 64 i + 63 of the staged rows
        const int idx = 64 * i + l, r = idx / nch, c = idx - r * nch;
        dma16(base, (uint32_t)(((int64_t)(row_of(r) - r0) * a.tab_rs + 8 * c) * 2), lds_addr(lds + 1024 * i));
    }
}

// rope_tab_load's entries of staged row r
__device__ __forceinline__ RopeTab rope_tab_lds(const uint8_t* lds, int r, int L, int rot) {
    RopeTab t;
    const int hc = rot >> 4;
    const int pc = L < hc ? L : (L < 2 * hc ? L - hc : 0);
    const uint8_t* src = lds + r * 4 * rot + 64 * pc + (L >= hc && L < 2 * hc ? 4 : 0);
#pragma unroll
    for (int j = 0; j < 8; ++j) t.w[j] = *reinterpret_cast<const uint32_t*>(src + 8 * j);
    return t;
}

// the lane's 8 weights (bf16 [128]) as floats
__device__ __forceinline__ void rope_w_load(const uint16_t* w, int L, float (&wv)[8]) { load8(w + 8 * L, wv); }

__device__ __forceinline__ float bf16_round(float x) { return (float)(bf16)x; }

__device__ __forceinline__ void h3_rms_rope(float (&x)[8], int L, const float (&w)[8], const RopeTab& t, int rot,
                                            float eps) {
    double ss = 0.0;
#pragma unroll
    for (int c = 0; c < 8; ++c) ss = fma((double)x[c], (double)x[c], ss);
    ss += xor_lane<1>(ss);
    ss += xor_lane<2>(ss);
    ss += xor_lane<4>(ss);
    ss += xor_lane<8>(ss);
    norm_bf16_exact8(x, 1.0 / sqrt(ss / 128.0 + (double)eps), w);
    const int hc = rot >> 4;
    const bool first = L < hc, second = L >= hc && L < 2 * hc;
    const int partner = first ? L + hc : (second ? L - hc : L);
    // first half: f00 x_i + f01 x_{i+rot/2} (own value x_i); second half: f10 x_i + f11 x_{i+rot/2} (own value
    // x_{i+rot/2}): with the second half's (f10, f11) swapped once, both are (own coefficient) * own + (partner's
    // coefficient) * partner. Both products are exact (bf16 times bf16), so the one rounding of the fma is the exact
    // sum's whichever product it takes.
    const uint32_t sel = first ? 0x03020100u : 0x01000302u;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const float y = __shfl(x[c], partner, 16);
        const uint32_t w = __builtin_amdgcn_perm(t.w[c], t.w[c], sel);
        const float yo = fmaf(lo_bf16(w), x[c], hi_bf16(w) * y);
        x[c] = first || second ? bf16_round(yo) : x[c];
    }
}

// ------------------------------------------------------------------------------------------------ prep launch 1
// Blocks x < nvchunk: channel abs-max of V over keys [x * 256, x * 256 + 256) of kv head y -> vpart.
// Block x == nvchunk: the anchor of kv head y (nine sample keys at i * (Sk - 1) / 8; the sample with the least
// squared distance to the others is subtracted from every key when that lowers the samples' energy and raises their
// abs-max by at most 12.5 %), in fp64 like the checker.
template <bool ROPE, int HD>
__global__ __launch_bounds__(256) void i8_stats_kernel(PrepArgs a) {
#pragma clang fp contract(off)
    constexpr int D = HD;
    constexpr int CGS = HD / 8, RPP = 256 / CGS;  // 8-channel groups a row; rows a pass
    constexpr int NSAMP = 9;
    // the V blocks' partial maxima and the anchor block's sums and sample rows share one buffer
    constexpr int RED_BYTES = RPP * HD * 4, SD_BYTES = (NSAMP + 2) * 128 * 8, ROWS_BYTES = ROPE ? NSAMP * 128 * 4 : 0;
    __shared__ __attribute__((aligned(16))) uint8_t smem[RED_BYTES > SD_BYTES + ROWS_BYTES ? RED_BYTES
                                                                                            : SD_BYTES + ROWS_BYTES];
    const Plan& p = a.p;
    const int b = blockIdx.z, hk = blockIdx.y, t = threadIdx.x;
    if ((int)blockIdx.x < p.nvchunk) {
        float (*red)[HD] = reinterpret_cast<float (*)[HD]>(smem);
        const int cg = t % CGS, r0 = t / CGS;
        float m[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) m[j] = 0.0f;
        const int base = blockIdx.x * VCHUNK;
        const uint16_t* vb = a.v + b * a.v_sb + hk * a.v_sh + 8 * cg;
#pragma unroll
        for (int i = 0; i < VCHUNK / RPP; ++i) {   // every load of the lane in flight together
            const int row = base + r0 + RPP * i;
            if (row < a.Sk) {
                const u32x4 w = *reinterpret_cast<const u32x4*>(vb + (int64_t)row * a.v_sn);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    m[2 * j] = fmaxf(m[2 * j], fabsf(lo_bf16(w[j])));
                    m[2 * j + 1] = fmaxf(m[2 * j + 1], fabsf(hi_bf16(w[j])));
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) red[r0][8 * cg + j] = m[j];
        __syncthreads();
        if (t < D) {
            float mx = 0.0f;
#pragma unroll
            for (int r = 0; r < RPP; ++r) mx = fmaxf(mx, red[r][t]);
            float* vpart = reinterpret_cast<float*>(a.ws + p.vpart);
            vpart[((size_t)(b * a.HK + hk) * p.nvchunk + blockIdx.x) * D + t] = mx;
        }
        return;
    }
    // the anchor
    double (*sd)[128] = reinterpret_cast<double (*)[128]>(smem);
    double s[NSAMP];
    const uint16_t* kb = a.k + b * a.k_sb + hk * a.k_sh;
    // fused rmsRope: the sample rows normalised and rotated first (16 lanes a row, groups 0-8), exactly as quant_k
    // prepares every key row
    float (*rows)[128] = reinterpret_cast<float (*)[128]>(smem + SD_BYTES);
    if constexpr (ROPE) {
        const int grp = t >> 4, L = t & 15;
        if (grp < NSAMP) {
            const int row = (int)((int64_t)grp * (a.Sk - 1) / (NSAMP - 1));
            float x[8], wv[8];
            load8(kb + (int64_t)row * a.k_sn + 8 * L, x);
            rope_w_load(a.kw, L, wv);
            h3_rms_rope(x, L, wv, rope_tab_load(a, row, L), a.rope_rot, a.rope_eps);
#pragma unroll
            for (int c = 0; c < 8; ++c) rows[grp][8 * L + c] = x[c];
        }
        __syncthreads();
    }
    if (t < D) {
        double e = 0.0, mx = 0.0, sum = 0.0;
#pragma unroll
        for (int i = 0; i < NSAMP; ++i) {
            const int row = (int)((int64_t)i * (a.Sk - 1) / (NSAMP - 1));
            if constexpr (ROPE) s[i] = (double)rows[i][t];
            else s[i] = (double)bf16_bits_to_f32(kb[(int64_t)row * a.k_sn + t]);
            e += s[i] * s[i];
            mx = fmax(mx, fabs(s[i]));
            sum += s[i];
        }
        sd[0][t] = e;
        sd[1][t] = mx;
#pragma unroll
        for (int j = 0; j < NSAMP; ++j) {
            const double d = NSAMP * s[j] - sum;
            sd[2 + j][t] = d * d;
        }
    }
    __syncthreads();
    for (int st = D / 2; st > 0; st >>= 1) {
        if (t < st) {
            sd[1][t] = fmax(sd[1][t], sd[1][t + st]);
            sd[0][t] += sd[0][t + st];
#pragma unroll
            for (int j = 0; j < NSAMP; ++j) sd[2 + j][t] += sd[2 + j][t + st];
        }
        __syncthreads();
    }
    const double orig_e = sd[0][0], orig_m = sd[1][0];
    int best = 0;
    for (int j = 1; j < NSAMP; ++j)
        if (sd[2 + j][0] < sd[2 + best][0]) best = j;
    __syncthreads();
    if (t < D) {
        double be = 0.0, bm = 0.0;
#pragma unroll
        for (int i = 0; i < NSAMP; ++i) {
            const double r = s[i] - s[best];
            be += r * r;
            bm = fmax(bm, fabs(r));
        }
        sd[0][t] = be;
        sd[1][t] = bm;
    }
    __syncthreads();
    for (int st = D / 2; st > 0; st >>= 1) {
        if (t < st) {
            sd[0][t] += sd[0][t + st];
            sd[1][t] = fmax(sd[1][t], sd[1][t + st]);
        }
        __syncthreads();
    }
    const bool improves = sd[0][0] < orig_e && sd[1][0] <= orig_m * 1.125;
    if (t == 0)
        reinterpret_cast<int*>(a.ws + p.anchor)[b * a.HK + hk] =
            improves ? (int)((int64_t)best * (a.Sk - 1) / (NSAMP - 1)) : -1;
    // the anchor row as quant_k subtracts it (a bf16 value, exact in the double sample), zeros when there is none
    if (t < D)
        reinterpret_cast<uint16_t*>(a.ws + p.arow)[(size_t)(b * a.HK + hk) * D + t] =
            improves ? (uint16_t)(__float_as_uint((float)s[best]) >> 16) : (uint16_t)0;
}

// ------------------------------------------------------------------------------------------------ prep launch 2
// Rows are read 16 bytes (8 channels) a lane, HD / 8 lanes a row.
constexpr int QROWS = 64;  // query rows per block
constexpr int KROWS = 64;  // key rows per block: four scale groups of 16, one per wave

// The 8 bf16 values of a lane's 16-byte row piece as floats
__device__ __forceinline__ void unpack8(const u32x4& w, float (&x)[8]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        x[2 * j] = lo_bf16(w[j]);
        x[2 * j + 1] = hi_bf16(w[j]);
    }
}

// Q: QROWS rows of head h per block, 256 / LPR per pass, one scale per row. Every row of the lane is in flight before
// the first is used (kept as bf16 until then); rows past Sq read row Sq - 1 and are zeroed.
template <int ROT, int HD, bool ROPE>
__device__ void quant_q(const PrepArgs& a, int b, int h, int qb, uint8_t* lds) {
#pragma clang fp contract(off)
    constexpr int LPR = HD / 8, RPB = 256 / LPR, NR = QROWS / RPB;  // lanes a row, rows a block pass, rows a lane
    const Plan& p = a.p;
    const int t = threadIdx.x, slot = t / LPR, L = t % LPR;
    const uint16_t* qbase = a.q + b * a.q_sb + h * a.q_sh + 8 * L;
    if constexpr (ROPE) rope_tab_dma(a, lds, [&](int r) { return min(qb * QROWS + r, a.Sq - 1); });
    u32x4 raw[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i)
        raw[i] = *reinterpret_cast<const u32x4*>(qbase + (int64_t)min(qb * QROWS + RPB * i + slot, a.Sq - 1) * a.q_sn);
    float wv[8];
    if constexpr (ROPE) {
        rope_w_load(a.qw, L, wv);
        LR_I8_WAIT_VMCNT(0);   // the table rows (and the lane's own loads)
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int row = qb * QROWS + RPB * i + slot;
        const bool ok = row < a.Sq;
        float x[8];
        unpack8(raw[i], x);
#pragma unroll
        for (int c = 0; c < 8; ++c) x[c] = ok ? x[c] : 0.0f;
        if constexpr (ROPE) h3_rms_rope(x, L, wv, rope_tab_lds(lds, RPB * i + slot, L, a.rope_rot), a.rope_rot, a.rope_eps);
        rotate8<ROT>(x, L);
        float m = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; ++c) m = fmaxf(m, fabsf(x[c]));
        const float mx = max_row<LPR>(m);
        const float sc = mx / 127.0f + 1e-7f;
        const float inv = 1.0f / sc;
        if (ok) {
            const size_t r = (size_t)(b * a.H + h) * a.Sq + row;
            *reinterpret_cast<u32x2*>(a.ws + p.q8 + r * HD + 8 * L) = pack_s8x8(x, inv);
            if (L == 0) reinterpret_cast<float*>(a.ws + p.qs)[r] = sc;
        }
    }
}

// K: KROWS key rows of kv head hk per block, 256 / LPR rows a pass (row RPB pass + t / LPR), four scale groups of 16
// rows; each wave's rows of a pass lie in one group, a group spans WPG waves. The anchor row (written by the stats
// launch: zeros when there is none) is subtracted before the rotation. The passes run two at a time: the lane keeps
// two rotated rows while the group maxima are combined across waves through LDS.
template <int ROT, int HD, bool ROPE>
__device__ void quant_k(const PrepArgs& a, int b, int hk, int kb, uint8_t* lds) {
#pragma clang fp contract(off)
    constexpr int LPR = HD / 8, RPW = 64 / LPR, RPB = 256 / LPR;  // lanes a row, rows a wave, rows a block pass
    constexpr int NPASS = KROWS / RPB, WPG = KGROUP / RPW;        // passes (4 or 2), waves a group (4 or 2)
    static_assert(NPASS % 2 == 0 && KGROUP % RPW == 0, "passes run in pairs; a wave's rows lie in one group");
    __shared__ float gmax[KROWS / KGROUP][4];   // [group][wave within the group]
    const Plan& p = a.p;
    const int t = threadIdx.x, wave = t >> 6, prow = t / LPR, L = t % LPR;
    const uint16_t* kbase = a.k + b * a.k_sb + hk * a.k_sh + 8 * L;
    // Rows past Sk (the last tile's padding) repeat real keys: those of the last key's scale group gL, key Sk - 1
    // standing in past its end. A padded row of group gL then equals key Sk - 1 and leaves the group's scale as it
    // is; a wholly padded group is a copy of group gL, scale included. Their scores equal real scores, so they never
    // raise a row max; the attention zeroes their P.
    const int last = a.Sk - 1, gl = last / KGROUP;
    auto src_of = [&](int row) { return row <= last ? row : min(gl * KGROUP + (row & (KGROUP - 1)), last); };
    if constexpr (ROPE) rope_tab_dma(a, lds, [&](int r) { return src_of(kb * KROWS + r); });
    u32x4 raw[NPASS];
#pragma unroll
    for (int i = 0; i < NPASS; ++i)  // all the lane's rows in flight before the first is used
        raw[i] = *reinterpret_cast<const u32x4*>(kbase + (int64_t)src_of(kb * KROWS + RPB * i + prow) * a.k_sn);
    float av[8], wv[8];
    load8(reinterpret_cast<const uint16_t*>(a.ws + p.arow) + (size_t)(b * a.HK + hk) * HD + 8 * L, av);
    if constexpr (ROPE) {
        rope_w_load(a.kw, L, wv);
        LR_I8_WAIT_VMCNT(0);   // the table rows (and the lane's own loads)
        __syncthreads();
    }
    uint8_t* k8 = a.ws + p.k8 + (size_t)(b * a.HK + hk) * p.skp * HD;
    float* aux_ks = reinterpret_cast<float*>(a.ws + p.aux + (size_t)(b * a.HK + hk) * p.ntiles * AUX_BYTES + AUX_KS_OFF);
#pragma unroll
    for (int ph = 0; ph < NPASS; ph += 2) {
        float x[2][8];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int lr = RPB * (ph + j) + prow;   // row within the block
            unpack8(raw[ph + j], x[j]);
            if constexpr (ROPE) h3_rms_rope(x[j], L, wv, rope_tab_lds(lds, lr, L, a.rope_rot), a.rope_rot, a.rope_eps);
#pragma unroll
            for (int c = 0; c < 8; ++c) x[j][c] = x[j][c] - av[c];
            rotate8<ROT>(x[j], L);
            float m = 0.0f;
#pragma unroll
            for (int c = 0; c < 8; ++c) m = fmaxf(m, fabsf(x[j][c]));
            m = max64(m);
            if ((t & 63) == 0) gmax[lr / KGROUP][wave % WPG] = m;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int lr = RPB * (ph + j) + prow, g = lr / KGROUP;
            float mx = gmax[g][0];
#pragma unroll
            for (int w = 1; w < WPG; ++w) mx = fmaxf(mx, gmax[g][w]);
            const float sc = mx / 127.0f + 1e-7f;
            const float inv = 1.0f / sc;
            const int row = kb * KROWS + lr;
            *reinterpret_cast<u32x2*>(k8 + (size_t)row * HD + 16 * ((L >> 1) ^ k_swz(row & 31, HD)) + 8 * (L & 1)) =
                pack_s8x8(x[j], inv);
            if (t % (64 * WPG) == 0) {   // the group's first wave, lane 0
                const int grp = kb * (KROWS / KGROUP) + g;
                const int tile = grp * KGROUP / p.cta, local = grp * KGROUP - tile * p.cta;
                aux_ks[(size_t)tile * (AUX_BYTES / 4) + ((local >> 4) & 1) * (p.cta / 32) + (local >> 5)] = sc;
            }
        }
    }
}

// V: one tile of cta keys of kv head hk per block: per-channel scales from the abs-max partials, int8, transposed into
// [HD dims][cta keys] in LDS (rows padded by 4 bytes, so that the lanes of a wave, which write different dims, spread
// over the banks), column sums per half tile into the aux block, then stored swizzled.
// ext: the kernel's own LDS buffer to use (the fused-rmsRope kernel shares one with the table staging), else null.
constexpr int VTS_BYTES = 128 * (128 + 4);
template <int HD, bool EXT>
__device__ void quant_v(const PrepArgs& a, int b, int hk, int tile, uint8_t* ext) {
#pragma clang fp contract(off)
    constexpr int CG = HD / 8, KQP = 256 / CG;  // 8-channel groups a key; key quads a block pass
    __shared__ float inv_own[EXT ? 1 : HD];
    __shared__ __attribute__((aligned(16))) uint8_t vts_own[EXT ? 1 : HD * (128 + 4)];
    uint8_t* vts = EXT ? ext : vts_own;
    float* inv_s = EXT ? reinterpret_cast<float*>(ext + VTS_BYTES) : inv_own;
    const Plan& p = a.p;
    const int cta = p.cta, vs = cta + 4, t = threadIdx.x;
    const size_t bhk = (size_t)b * a.HK + hk;
    if (t < HD) {
        const float* vpart = reinterpret_cast<const float*>(a.ws + p.vpart) + bhk * p.nvchunk * HD;
        float mx = 0.0f;
        for (int c = 0; c < p.nvchunk; ++c) mx = fmaxf(mx, vpart[c * HD + t]);
        const float sc = fmaxf(mx * (1.0f / 127.0f), 1e-12f);
        inv_s[t] = 1.0f / sc;
        if (tile == 0) reinterpret_cast<float*>(a.ws + p.vs)[bhk * HD + t] = sc;
    }
    __syncthreads();
    const int c8 = t % CG, k0 = t / CG;  // channels 8 c8 .. + 7; key quads k0, k0 + KQP, ...
    float inv[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) inv[c] = inv_s[8 * c8 + c];
    const uint16_t* vb = a.v + b * a.v_sb + hk * a.v_sh + 8 * c8;
    for (int kq = k0; kq < cta / 4; kq += KQP) {  // keys 4 kq .. 4 kq + 3 of the tile
        u32x4 raw[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {  // the four keys in flight together
            const int key = tile * cta + 4 * kq + r;
            raw[r] = key < a.Sk ? *reinterpret_cast<const u32x4*>(vb + (int64_t)key * a.v_sn) : u32x4{0u, 0u, 0u, 0u};
        }
        // (keys past Sk arrive as zero rows: their bytes are 0)
        uint32_t col[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int lo[4], hi[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                lo[r] = rn_sat(lo_bf16(raw[r][j]) * inv[2 * j]);
                hi[r] = rn_sat(hi_bf16(raw[r][j]) * inv[2 * j + 1]);
            }
            col[2 * j] = pack_lo_bytes(lo[0], lo[1], lo[2], lo[3]);
            col[2 * j + 1] = pack_lo_bytes(hi[0], hi[1], hi[2], hi[3]);
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) *reinterpret_cast<uint32_t*>(vts + (8 * c8 + c) * vs + 4 * kq) = col[c];
    }
    __syncthreads();
    uint8_t* aux = a.ws + p.aux + (bhk * p.ntiles + tile) * AUX_BYTES;
    if (t < 2 * HD) {
        const int d = t % HD, half = t / HD;
        int s = 0;
        for (int w = 0; w < cta / 8; ++w)
            s = __builtin_amdgcn_sdot4(*reinterpret_cast<const int*>(vts + d * vs + half * (cta / 2) + 4 * w),
                                       0x01010101, s, false);
        reinterpret_cast<int16_t*>(aux)[(half * 32 + (d & 31)) * (HD / 32) + (d >> 5)] = (int16_t)s;
    }
    uint8_t* vt = a.ws + p.vt + (bhk * p.ntiles + tile) * (size_t)(HD * cta);
    const int cpr = cta / 16;  // chunks per dim row
    for (int idx = t; idx < HD * cpr; idx += 256) {
        const int d = idx / cpr, c = idx - d * cpr;
        const uint32_t* src = reinterpret_cast<const uint32_t*>(vts + d * vs + 16 * c);
        const u32x4 w = {src[0], src[1], src[2], src[3]};
        *reinterpret_cast<u32x4*>(vt + d * cta + 16 * (c ^ v_swz(d, cta))) = w;
    }
}

// Dynamic LDS of the fused-rmsRope instantiations: the staged table rows (Q and K blocks) or quant_v's arrays (V).
inline size_t quant_lds_bytes(int rot) {
    const size_t t = tab_lds_bytes(rot), v = VTS_BYTES + 4 * 128;
    return t > v ? t : v;
}

// grid (ceil(Sq / QROWS) + skp / KROWS + ntiles, max(H, HK), B): Q blocks, then K blocks, then V tiles. The
// fused-rmsRope instantiations run with quant_lds_bytes(rope_rot) bytes of dynamic LDS.
template <int ROT, int HD, bool ROPE = false>
__global__ __launch_bounds__(256) void i8_quant_kernel(PrepArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int b = blockIdx.z, y = blockIdx.y;
    const int nqb = (a.Sq + QROWS - 1) / QROWS, nkb = a.p.skp / KROWS;
    int x = blockIdx.x;
    if (x < nqb) {
        if (y < a.H) quant_q<ROT, HD, ROPE>(a, b, y, x, lds);
        return;
    }
    x -= nqb;
    if (x < nkb) {
        if (y < a.HK) quant_k<ROT, HD, ROPE>(a, b, y, x, lds);
        return;
    }
    x -= nkb;
    if (y < a.HK) quant_v<HD, ROPE>(a, b, y, x, lds);
}

// ------------------------------------------------------------------------------------------------ attention
// A workgroup barrier that neither waits for outstanding memory operations nor lets the compiler move any
// instruction across it (the waits that matter are issued explicitly; the clusters on either side stay apart).
__device__ __forceinline__ void block_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

__device__ __forceinline__ float pair_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float pair_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Key (within a 32-key block) held by MFMA row m: bits (b4 b3 b2 b1 b0) -> (b2 b4 b3 b1 b0), so that score register
// r of lane half h is key 16 h + r.
__device__ __forceinline__ int key_perm(int m) {
    return (m & 3) | (((m >> 3) & 1) << 2) | (((m >> 4) & 1) << 3) | (((m >> 2) & 1) << 4);
}

// a ^ b on the VALU, opaque to the optimiser: keeps per-fragment LDS addresses from being precomputed and held in
// registers across the loop (they are one XOR away from a per-stage base). b is wave-uniform.
__device__ __forceinline__ uint32_t xor_opaque(uint32_t a, uint32_t b) {
    if (b == 0) return a;
    uint32_t r;
    asm volatile("v_xor_b32 %0, %1, %2" : "=v"(r) : "s"(b), "v"(a));
    return r;
}

template <typename T>
__device__ __forceinline__ T lds_at(uint32_t addr) {
    return *reinterpret_cast<const __attribute__((address_space(3))) T*>((uintptr_t)addr);
}

template <typename T>
__device__ __forceinline__ T lds_load(const uint8_t* p) {
    return *reinterpret_cast<const __attribute__((address_space(3))) T*>(
        (__attribute__((address_space(3))) const uint8_t*)p);
}

// Accumulators start at this bias instead of 0: an int32 accumulator a with |a - MAGIC| < 2^22 read as an fp32 is
// exactly 12582912 + (a - MAGIC), so no int -> float conversion is needed; the bias is taken out by the same FMA
// (scores) or by the column-sum MFMA (P V).
constexpr int MAGIC = 0x4B400000;
constexpr float MAGF = 12582912.0f;
constexpr float LAZY = 64.0f;

// One workgroup: 8 waves x 32 queries. Per key tile t a wave runs two phases, each an explicit slot schedule (one
// MFMA per slot; a sched_barrier closes every slot, so its VALU work stays with it):
//   A: S(t+1) = K(t+1) Q^T (int8 MFMA, two 32-key accumulator chains alternating), and in the same slots P(t) from
//      S(t): x = s * c - m_t (one FMA on the biased score), P = exp2(x) to u8, its row sum (udot4), P ^ 0x80;
//   B: O^T += V(t)^T P(t) (int8 MFMA, one 32-dim block after the other, two accumulators alternating), and in the
//      same slots the fp32 update of the previous block, O += ts * acc, and the row max of S(t+1);
//   operand fragments are read from LDS two slots ahead;
//   then the column-sum correction (one f32 MFMA per 32-dim block) and tile t+1's constants (max, scales).
// K, V^T and the aux block of tile t+3 are loaded into a 4-stage LDS ring while tiles t and t+1 are read.
// A workgroup below a.nwhole computes one query block over all key tiles and writes its rows; one at or past it (a
// piece) computes a block of the last partial round over its key range [t0, t1) and leaves the unnormalised rows and
// (reference, row sum) in the partial area for i8_split_combine_kernel.
template <int CTA, int NS, int HD>
__global__ __launch_bounds__(512, 1) __attribute__((amdgpu_waves_per_eu(2, 2))) void i8_attn_kernel(AttnArgs a) {
    constexpr int NB = CTA / 32;                   // 32-key blocks per tile
    constexpr int DB = HD / 32;                    // 32-dim blocks of a row (and k-steps of a score MFMA chain)
    constexpr int TB = CTA * HD;                   // bytes of a K (or V^T) tile
    constexpr int STAGE = 2 * TB + AUX_BYTES;
    constexpr int NW = 8;                          // waves per workgroup, 32 queries each
    constexpr int NBLK = TB / 1024;                // 1 KB direct loads per K (or V^T) tile
    constexpr int KVL = NBLK >= NW ? NBLK / NW : 0;  // ... per wave, when every wave loads K and V alike
    // this wave's direct loads per tile (with NBLK = NW / 2 each wave loads one block: waves 0-3 K, 4-7 V)
    constexpr int LPT = KVL > 0 ? 2 * KVL : 1;
    constexpr int QS = DB * NB;                    // score MFMAs per tile (NB blocks x DB dim steps)
    constexpr int PS = DB * NB;                    // P V MFMAs per tile (DB dim blocks x NB key steps)
    constexpr int SPM = 4 * NB / QS;               // phase-A slots (P dwords) per score MFMA
    static_assert(NS == 4 && (KVL > 0 || 2 * NBLK == NW) && 4 * NB % QS == 0, "the ring and slot schedules");
    __shared__ __attribute__((aligned(1024))) uint8_t ring[NS * STAGE];

    const Plan& p = a.p;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 31, hf = lane >> 5;

    // Whole blocks (workgroups below nwhole) in XCD-aware order: consecutive logical blocks (same head) land on the
    // same XCD and share its L2. Pieces: workgroup nwhole + P i + r takes key tiles [r T / P, (r + 1) T / P) of block
    // nwhole + i, with the cuts rounded to the nearest multiple of NS (cuts at least NS apart: T >= NS P).
    const int bx = blockIdx.x;
    const bool piece = bx >= a.nwhole;
    int logical, t0 = 0, t1 = p.ntiles;
    if (!piece) {
        const int nwg = a.nwhole, per = nwg >> 3, rem = nwg & 7, xcd = bx & 7, idx = bx >> 3;
        logical = xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
    } else {
        const int i = (bx - a.nwhole) / a.P, r = bx - a.nwhole - i * a.P;
        logical = a.nwhole + i;
        t0 = (r * p.ntiles / a.P + NS / 2) / NS * NS;
        t1 = r + 1 == a.P ? p.ntiles : ((r + 1) * p.ntiles / a.P + NS / 2) / NS * NS;
    }
    const int nqb = (a.Sq + 255) / 256;
    const int qblk = logical % nqb, bh = logical / nqb;
    const int head = bh % a.H, b = bh / a.H;
    const int hk = head / a.G;
    const size_t bhk = (size_t)b * a.HK + hk;

    const uint8_t* k8 = a.ws + p.k8 + bhk * p.skp * HD;
    const uint8_t* vt = a.ws + p.vt + bhk * p.skp * HD;
    const uint8_t* aux = a.ws + p.aux + bhk * p.ntiles * AUX_BYTES;
    const int ntiles = p.ntiles;
    const int tail = a.Sk - (ntiles - 1) * CTA;  // valid keys of the last tile

    // queries: B operand fragments (dims 32 s + 16 hf .. + 15) and the row scale
    const int q = qblk * 256 + wave * 32 + n;
    const bool qok = q < a.Sq;
    const size_t qr = (size_t)(b * a.H + head) * a.Sq + (qok ? q : a.Sq - 1);
    i32x4 Qf[DB];
    {
        const uint8_t* src = a.ws + p.q8 + qr * HD + 16 * hf;
#pragma unroll
        for (int s = 0; s < DB; ++s) Qf[s] = qok ? *reinterpret_cast<const i32x4*>(src + 32 * s) : i32x4{0, 0, 0, 0};
    }
    const float cq = (qok ? reinterpret_cast<const float*>(a.ws + p.qs)[qr] : 1.0f) * a.c;

    // Fragment addresses: chunk (2 s + hf) ^ x of a row is chunk hf ^ x with bits 5-6 of the byte address flipped by
    // 32 s (every other address term has those bits clear), so each fragment is one XOR from a per-stage base.
    const int kp = key_perm(n), kx = k_swz(kp, HD), vx = v_swz(n, CTA);
    const uint32_t k_lane = (uint32_t)(kp * HD + 16 * (hf ^ kx));
    const uint32_t v_lane = (uint32_t)(TB + n * CTA + 16 * (hf ^ vx));
    // score MFMA f of a tile: two 32-key blocks' chains alternate, each over the DB dim steps
    auto kb_of = [](int f) { return 2 * (f / (2 * DB)) + (f & 1); };
    auto ks_of = [](int f) { return (f >> 1) % DB; };
    auto kfrag = [&](const uint8_t* st, int f) -> i32x4 {
        return lds_at<i32x4>(xor_opaque(lds_addr(st) + k_lane, 32 * ks_of(f)) + 32 * HD * kb_of(f));
    };
    auto vfrag = [&](const uint8_t* st, int f) -> i32x4 {  // P V MFMA f: dim block f / NB, key step f % NB
        const int bb = f / NB, j = f % NB;
        return lds_at<i32x4>(xor_opaque(lds_addr(st) + v_lane, 32 * j) + 32 * CTA * bb);
    };

    // ring stage of tile t (a piece's first tile t0 is a multiple of NS: its ring starts at stage 0 too)
    auto stage = [&](int t) { return ring + (t % NS) * STAGE; };
    auto issue = [&](int t) {
        uint8_t* st = stage(t);
        if constexpr (KVL > 0) {
#pragma unroll
            for (int i = 0; i < KVL; ++i) {
                const int blk = wave * KVL + i;
                dma16(k8 + (size_t)t * TB + blk * 1024, lane * 16, lds_addr(st + blk * 1024));
                dma16(vt + (size_t)t * TB + blk * 1024, lane * 16, lds_addr(st + TB + blk * 1024));
            }
        } else if (wave < NBLK) {
            dma16(k8 + (size_t)t * TB + wave * 1024, lane * 16, lds_addr(st + wave * 1024));
        } else {
            dma16(vt + (size_t)t * TB + (wave - NBLK) * 1024, lane * 16, lds_addr(st + TB + (wave - NBLK) * 1024));
        }
        if (wave == 0) dma16(aux + (size_t)t * AUX_BYTES, lane * 16, lds_addr(st + 2 * TB));
    };
    // wait until tile `need` has landed, given that tiles up to `issued` were issued
    auto wait_for = [&](int need, int issued) {
        const bool one = issued > need;  // at most one later tile (NS = 4: issued <= need + 1)
        if (wave == 0) {
            if (one) LR_I8_WAIT_VMCNT(LPT + 1);
            else LR_I8_WAIT_VMCNT(0);
        } else {
            if (one) LR_I8_WAIT_VMCNT(LPT);
            else LR_I8_WAIT_VMCNT(0);
        }
    };

    i32x16 magic;
#pragma unroll
    for (int r = 0; r < 16; ++r) magic[r] = MAGIC;
    f32x16 O[DB];
#pragma unroll
    for (int bb = 0; bb < DB; ++bb)
#pragma unroll
        for (int r = 0; r < 16; ++r) O[bb][r] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f, ts = 0.0f;
    float cc[NB], nbias[NB];

    // tile constants from the biased int row maxima mi of a tile's scores (K scales from its aux block):
    // c = q_scale * k_scale * scale * log2(e) per 16-key group, m_t = tile max - log2(255), the row's reference m_run
    // and the two scales, then the per-block FMA bias -(12582912 c + m_t) that takes out the accumulator bias too.
    // The reference moves only when a tile's m_t passes it by more than LAZY (log2 units): a tile then enters O with
    // weight ts = 2^(m_t - m_run) <= 2^LAZY, so O stays below 2^64 * 255 * 127 * cta * ntiles (far from the fp32
    // range) and the rescale of O, which a running maximum would need on most tiles, is rare. O / l is the same
    // softmax: every tile's weight relative to any fixed reference cancels in the quotient.
    auto constants = [&](const int (&mi)[NB], const uint8_t* st) {
        const uint8_t* ksp = st + 2 * TB + AUX_KS_OFF + 4 * NB * hf;
        float tmx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < NB; ++kb) {
            cc[kb] = cq * lds_load<float>(ksp + 4 * kb);
            tmx = fmaxf(tmx, (__int_as_float(mi[kb]) - MAGF) * cc[kb]);
        }
        tmx = pair_max(tmx) - S_U8_OFFSET;
        const float m_new = tmx > m_run + LAZY ? tmx : m_run;
        const float os = __builtin_amdgcn_exp2f(m_run - m_new);
        ts = __builtin_amdgcn_exp2f(tmx - m_new);
        m_run = m_new;
#pragma unroll
        for (int kb = 0; kb < NB; ++kb) nbias[kb] = -fmaf(MAGF, cc[kb], tmx);
        if (__builtin_amdgcn_ballot_w64(os != 1.0f) != 0) {
            l_run *= os;
#pragma unroll
            for (int bb = 0; bb < DB; ++bb)
#pragma unroll
                for (int r = 0; r < 16; ++r) O[bb][r] *= os;
        }
    };
    auto rowmax = [&](const i32x16 (&S)[NB], int (&mi)[NB]) {
#pragma unroll
        for (int kb = 0; kb < NB; ++kb) {
            mi[kb] = S[kb][0];
#pragma unroll
            for (int r = 1; r < 16; ++r) mi[kb] = max(mi[kb], S[kb][r]);
        }
    };

    // prologue: tiles t0 .. t0 + NS-2 in flight, S(t0) and its constants
#pragma unroll
    for (int j = 0; j < NS - 1; ++j)
        if (t0 + j < t1) issue(t0 + j);
    wait_for(1, min(NS - 2, t1 - t0 - 1));
    block_barrier();
    i32x16 SS[2][NB];  // S(t) in SS[t & 1]
    {
#pragma unroll
        for (int kb = 0; kb < NB; ++kb) SS[0][kb] = magic;
#pragma unroll
        for (int f = 0; f < QS; ++f)
            SS[0][kb_of(f)] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kfrag(ring, f), Qf[ks_of(f)], SS[0][kb_of(f)], 0, 0, 0);
        int mi[NB];
        rowmax(SS[0], mi);
        constants(mi, ring);
    }

    // One key tile: S holds S(t); NEXT: S(t+1) is computed into Sn in phase A (every tile but the last); LAST: tile t
    // is the last one (P of keys past Sk zeroed when it is partial). A partial last tile needs no mask for its row
    // max: the prep fills its key rows past Sk with duplicates of real keys (same int8 row, same scale), which never
    // exceed the max. The two score arrays swap roles from tile to tile (the loop below takes tiles in pairs), so no
    // registers are copied.
    auto step = [&](int t, auto par_c, auto next_c, auto last_c) {
        constexpr int PAR = decltype(par_c)::value;
        constexpr bool NEXT = decltype(next_c)::value;
        constexpr bool LAST = decltype(last_c)::value;
        i32x16 (&S)[NB] = SS[PAR];
        i32x16 (&Sn)[NB] = SS[PAR ^ 1];
        if (t + NS - 1 < t1) issue(t + NS - 1);
        const uint8_t* stK = stage(t + 1);
        const uint8_t* stV = stage(t);
        const bool mask_p = LAST && t1 == ntiles && tail < CTA;

        // ---- phase A: S(t+1) on MFMA, P(t) on VALU
        uint32_t P[NB][4];
        uint32_t rs = 0;
        i32x4 fr[3];
        if (NEXT) {
            fr[0] = kfrag(stK, 0);
            fr[1] = kfrag(stK, 1);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < 4 * NB; ++s) {
            if (NEXT && s % SPM == 0) {  // score MFMA f in the first slot of its group of SPM
                const int f = s / SPM;
                if (f + 2 < QS) fr[(f + 2) % 3] = kfrag(stK, f + 2);
                const int kb = kb_of(f), ks = ks_of(f);
                Sn[kb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fr[f % 3], Qf[ks], ks == 0 ? magic : Sn[kb], 0, 0, 0);
            }
            {
                const int kb = s >> 2, qd = s & 3;  // P dword s: block kb, keys 16 hf + 4 qd .. + 3
                uint32_t w = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float e = __builtin_amdgcn_exp2f(fmaf(__int_as_float(S[kb][4 * qd + i]), cc[kb], nbias[kb]));
                    w = __builtin_amdgcn_cvt_pk_u8_f32(e, i, w);
                }
                if (mask_p) {
                    uint32_t keep = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (32 * kb + 16 * hf + 4 * qd + i < tail) keep |= 0xffu << (8 * i);
                    w &= keep;
                }
                rs = __builtin_amdgcn_udot4(w, 0x01010101u, rs, false);
                P[kb][qd] = w ^ 0x80808080u;
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        l_run = fmaf(ts, (float)rs, l_run);

        // ---- phase B: O^T += V(t)^T P(t) on MFMA; the previous block's fp32 update and the max of S(t+1) on VALU
        int mi[NB];
#pragma unroll
        for (int kb = 0; kb < NB; ++kb) mi[kb] = MAGIC - (1 << 22);
        i32x16 acc[2];
        fr[0] = vfrag(stV, 0);
        fr[1] = vfrag(stV, 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < PS; ++s) {
            if (s + 2 < PS) fr[(s + 2) % 3] = vfrag(stV, s + 2);
            const int bb = s / NB, j = s % NB;
            const i32x4 B = {(int)P[j][0], (int)P[j][1], (int)P[j][2], (int)P[j][3]};
            acc[bb & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fr[s % 3], B, j == 0 ? magic : acc[bb & 1], 0, 0, 0);
            if (NEXT) {  // max of S(t+1): its NB * 16 registers spread evenly over the PS slots
                static_assert(NB * 16 % (4 * PS) == 0, "whole groups of 4 registers per slot");
#pragma unroll
                for (int u = 0; u < NB * 16 / PS / 4; ++u) {
                    const int g = (NB * 16 / PS) * s + 4 * u;  // flat register index kb * 16 + r, < NB * 16
                    const int kb = g >> 4, r = g & 15;
                    mi[kb] = max(max(mi[kb], Sn[kb][r]), max(max(Sn[kb][r + 1], Sn[kb][r + 2]), Sn[kb][r + 3]));
                }
            }
            if (bb >= 1) {  // fp32 update of block bb - 1, spread over block bb's slots
                const int pb = bb - 1;
#pragma unroll
                for (int u = 0; u < 16 / NB; ++u) {
                    const int r = j * (16 / NB) + u;
                    O[pb][r] = fmaf(__int_as_float(acc[pb & 1][r]), ts, O[pb][r]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) O[DB - 1][r] = fmaf(__int_as_float(acc[(DB - 1) & 1][r]), ts, O[DB - 1][r]);
        {
            // + 128 * ts * (column sums of V(t)) - 12582912 * ts (the P V accumulator bias), per 32-dim block
            int16_t cs[DB];
            if constexpr (DB == 4) {
                const i16x4 c4 = lds_load<i16x4>(stV + 2 * TB + 8 * lane);
#pragma unroll
                for (int bb = 0; bb < 4; ++bb) cs[bb] = c4[bb];
            } else {
                const uint32_t c2 = lds_load<uint32_t>(stV + 2 * TB + 4 * lane);
                cs[0] = (int16_t)(c2 & 0xffffu);
                cs[1] = (int16_t)(c2 >> 16);
            }
            const float w128 = 128.0f * ts;
#pragma unroll
            for (int bb = 0; bb < DB; ++bb)
                O[bb] = __builtin_amdgcn_mfma_f32_32x32x2f32((float)cs[bb] - 49152.0f, w128, O[bb], 0, 0, 0);
        }
        if (NEXT) {
            constants(mi, stK);
            if (t + 2 < t1) wait_for(t + 2, min(t1 - 1, t + NS - 1));
            else LR_I8_WAIT_VMCNT(0);
            block_barrier();
        }
    };
    // the last tile (every load has landed: the wait before the previous barrier) has no S(t+1)
    int t = t0;
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    for (; t + 2 < t1; t += 2) {
        step(t, P0{}, std::true_type{}, std::false_type{});
        step(t + 1, P1{}, std::true_type{}, std::false_type{});
    }
    if (t + 1 < t1) {
        step(t, P0{}, std::true_type{}, std::false_type{});
        step(t + 1, P1{}, std::false_type{}, std::true_type{});
    } else {
        step(t, P0{}, std::false_type{}, std::true_type{});
    }

    if (!qok) return;
    const float* vs = reinterpret_cast<const float*>(a.ws + p.vs) + bhk * HD;
    if (piece) {   // the piece's unnormalised rows times the V scales, and (reference, row sum), to the partial area
        const int pc = bx - a.nwhole, ql = wave * 32 + n;
        float* po = a.part + ((size_t)pc * 256 + ql) * HD;
#pragma unroll
        for (int bb = 0; bb < DB; ++bb)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d0 = 32 * bb + 8 * g + 4 * hf;
                const f32x4 v = *reinterpret_cast<const f32x4*>(vs + d0);
                *reinterpret_cast<f32x4*>(po + d0) = f32x4{O[bb][4 * g] * v[0], O[bb][4 * g + 1] * v[1],
                                                           O[bb][4 * g + 2] * v[2], O[bb][4 * g + 3] * v[3]};
            }
        const float l = pair_sum(l_run);
        if (hf == 0) {
            float* pm = a.part + (size_t)p.part_n * 256 * HD + ((size_t)pc * 256 + ql) * 2;
            pm[0] = m_run;
            pm[1] = l;
        }
        return;
    }
    const float inv = 1.0f / pair_sum(l_run);
    uint16_t* orow = a.out + b * a.o_sb + head * a.o_sh + (int64_t)q * a.o_sn;
#pragma unroll
    for (int bb = 0; bb < DB; ++bb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d0 = 32 * bb + 8 * g + 4 * hf;
            const f32x4 v = *reinterpret_cast<const f32x4*>(vs + d0);
            u32x2 w;
            w[0] = pack_bf16x2(O[bb][4 * g] * inv * v[0], O[bb][4 * g + 1] * inv * v[1]);
            w[1] = pack_bf16x2(O[bb][4 * g + 2] * inv * v[2], O[bb][4 * g + 3] * inv * v[3]);
            *reinterpret_cast<u32x2*>(orow + d0) = w;
        }
}

// The rows of the split query blocks: one wave per query row, O = sum_r 2^(m_r - M) O_r / sum_r 2^(m_r - M) l_r over
// the block's P pieces (M = max_r m_r; every piece covers at least one key tile, so m_r is finite), two dims a lane.
template <int HD>
__global__ __launch_bounds__(256) void i8_split_combine_kernel(AttnArgs a) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int nqb = (a.Sq + 255) / 256;
    if (row >= (nqb * a.H * a.B - a.nwhole) * 256 || 2 * lane >= HD) return;
    const int i = row >> 8, ql = row & 255;
    const int blk = a.nwhole + i, qblk = blk % nqb, bh = blk / nqb, head = bh % a.H, b = bh / a.H;
    const int q = qblk * 256 + ql;
    if (q >= a.Sq) return;
    const float* ml = a.part + (size_t)a.p.part_n * 256 * HD;
    float M = -INFINITY;
    for (int r = 0; r < a.P; ++r) M = fmaxf(M, ml[((size_t)(i * a.P + r) * 256 + ql) * 2]);
    float L = 0.0f, o0 = 0.0f, o1 = 0.0f;
    for (int r = 0; r < a.P; ++r) {
        const size_t pr = (size_t)(i * a.P + r) * 256 + ql;
        const float w = __builtin_amdgcn_exp2f(ml[2 * pr] - M);
        L = fmaf(w, ml[2 * pr + 1], L);
        const float2 ov = *reinterpret_cast<const float2*>(a.part + pr * HD + 2 * lane);
        o0 = fmaf(w, ov.x, o0);
        o1 = fmaf(w, ov.y, o1);
    }
    const float inv = 1.0f / L;
    *reinterpret_cast<uint32_t*>(a.out + b * a.o_sb + head * a.o_sh + (int64_t)q * a.o_sn + 2 * lane) =
        pack_bf16x2(o0 * inv, o1 * inv);
}

template <int CTA, int HD>
void launch_blocks(const AttnArgs& a, unsigned grid, hipStream_t stream) {
    hipLaunchKernelGGL((i8_attn_kernel<CTA, 4, HD>), dim3(grid), dim3(512), 0, stream, a);
}

}  // namespace

hipError_t launch_prep(const PrepArgs& a, hipStream_t stream) {
    const Plan& p = a.p;
    const dim3 sgrid(p.nvchunk + 1, a.HK, a.B);
    if (a.rope_tab && p.d == 128) hipLaunchKernelGGL((i8_stats_kernel<true, 128>), sgrid, dim3(256), 0, stream, a);
    else if (a.rope_tab) return hipErrorInvalidValue;   // the fused rmsRope: head dim 128 only
    else if (p.d == 128) hipLaunchKernelGGL((i8_stats_kernel<false, 128>), sgrid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((i8_stats_kernel<false, 64>), sgrid, dim3(256), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const dim3 grid((a.Sq + QROWS - 1) / QROWS + p.skp / KROWS + p.ntiles, a.H > a.HK ? a.H : a.HK, a.B);
    if (a.rope_tab) {   // the fused rmsRope: head dim 128 only (checked by the caller)
        if (p.d != 128) return hipErrorInvalidValue;
        const size_t lds = quant_lds_bytes(a.rope_rot);
        if (p.rot == 4) hipLaunchKernelGGL((i8_quant_kernel<4, 128, true>), grid, dim3(256), lds, stream, a);
        else hipLaunchKernelGGL((i8_quant_kernel<128, 128, true>), grid, dim3(256), lds, stream, a);
    } else if (p.d == 128) {
        if (p.rot == 4) hipLaunchKernelGGL((i8_quant_kernel<4, 128>), grid, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((i8_quant_kernel<128, 128>), grid, dim3(256), 0, stream, a);
    } else {
        if (p.rot == 4) hipLaunchKernelGGL((i8_quant_kernel<4, 64>), grid, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((i8_quant_kernel<64, 64>), grid, dim3(256), 0, stream, a);
    }
    return hipGetLastError();
}

// One workgroup per query block of 256 rows. When the blocks leave a last round of at most half the compute units
// and there are at least 4 SPLIT_MAX key tiles, that round's blocks are cut into P key ranges each (P up to SPLIT_MAX,
// at most one piece per compute unit), and a second launch merges the pieces' rows.
hipError_t launch_attention(AttnArgs a, int cus, hipStream_t stream) {
    const int64_t nqb = (a.Sq + 255) / 256, nblk = nqb * a.H * a.B;
    if (nblk > 0x7fffffff / SPLIT_MAX) return hipErrorInvalidValue;
    a.nwhole = (int)nblk;
    a.P = 1;
    a.part = reinterpret_cast<float*>(a.ws + a.p.part);
    const int64_t rem = cus > 0 ? nblk % cus : 0;
    if (rem > 0 && 2 * rem <= cus && a.p.ntiles >= 4 * SPLIT_MAX) {
        const int P = (int)std::min<int64_t>(std::min<int64_t>(SPLIT_MAX, cus / rem), a.p.part_n / rem);
        if (P >= 2) {
            a.nwhole = (int)(nblk - rem);
            a.P = P;
        }
    }
    const unsigned grid = (unsigned)(a.nwhole + (nblk - a.nwhole) * a.P);
    if (a.p.d == 64) launch_blocks<64, 64>(a, grid, stream);
    else if (a.p.cta == 128) launch_blocks<128, 128>(a, grid, stream);
    else launch_blocks<64, 128>(a, grid, stream);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.P == 1) return e;
    const int64_t rows = (nblk - a.nwhole) * 256;
    if (a.p.d == 64)
        hipLaunchKernelGGL(i8_split_combine_kernel<64>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(i8_split_combine_kernel<128>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace i8
}  // namespace lr
