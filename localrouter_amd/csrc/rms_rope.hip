// Per-(token, head) RMSNorm + RoPE over bf16 rows, for gfx950.
//
// Semantics: kernels/cuda/minimax/kitchen/rms_rope.cu:37-230 with rope_device.cuh:65-98 (MiniMax H3: rrms =
// 1/sqrt(sum(x^2)/128 + eps), y = x * rrms * w, the normalised value rounded to bf16 before the rotation, pairs
// (i, i + rot/2) rotated by [f00 f01; f10 f11] from a bf16 table [rows][rot/2][2][2], dims >= rot norm-only) and the
// Qwen-Image form launched by src/engines/qwen_image/triton_k.zig:44-53 (fp32 weight, fp32 cos/sin [N, rot/2]).
//
// Layout of the work: a group of 16 lanes owns one token row and HPG heads of it; lane c holds dims 8c..8c+7 of each
// head as one 16-byte load. All loads of a group (its heads, the weight, the row's table entries) are issued before any
// of them is consumed, the table and weight are shared by the group's heads, the sum of squares is a 4-step xor
// butterfly inside the group, and a split-half partner chunk comes from lane c +- rot/16 of the same group. The table
// kind and the pairing are template parameters, so the loop bodies carry no per-element branches.
// HBM-bound by design: 256 bytes in and 256 bytes out per (row, head). The joint attention's query preparation is
// this pass with post_scale = scale * log2 e (the streaming kernel's exp2-domain scores).
#include "lr_common.h"
#include "lr_kernels.h"

namespace lr {

namespace {

constexpr int HPG = 4;   // heads per 16-lane group

// Rotation coefficients of pair p (clamped to a valid pair: callers select the result away for p >= rot/2).
template <int KIND>
__device__ __forceinline__ Rot2 rot_at(const void* ta, const void* tb, int64_t row_off, int p) {
    Rot2 r;
    if constexpr (KIND == TABLE_COSSIN_F32) {
        const float c = static_cast<const float*>(ta)[row_off + p];
        const float s = static_cast<const float*>(tb)[row_off + p];
        r.f00 = c; r.f01 = -s; r.f10 = s; r.f11 = c;
    } else if constexpr (KIND == TABLE_MAT2_BF16) {
        const u32x2 m = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(ta) + row_off + 4 * p);
        r.f00 = lo_bf16(m[0]); r.f01 = hi_bf16(m[0]); r.f10 = lo_bf16(m[1]); r.f11 = hi_bf16(m[1]);
    } else if constexpr (KIND == TABLE_MAT2_F32) {
        const f32x4 m = *reinterpret_cast<const f32x4*>(static_cast<const float*>(ta) + row_off + 4 * p);
        r.f00 = m[0]; r.f01 = m[1]; r.f10 = m[2]; r.f11 = m[3];
    } else {
        r.f00 = 1.0f; r.f01 = 0.0f; r.f10 = 0.0f; r.f11 = 1.0f;
    }
    return r;
}

template <int KIND, int PAIRING>
__global__ __launch_bounds__(256) void rms_rope_kernel(RopeArgs a) {
    const int tid = threadIdx.x;
    const int c = tid & 15;
    const int hgroups = (a.heads + HPG - 1) / HPG;
    const int64_t g = (int64_t)blockIdx.x * 16 + (tid >> 4);
    const int64_t total = a.rows * hgroups;
    const bool live = g < total;
    const int64_t gg = live ? g : total - 1;           // dead groups mirror the last one, then skip the stores
    const int64_t row = gg / hgroups;
    const int h0 = (int)(gg - row * hgroups) * HPG;

    // ---- every load first
    u32x4 xin[HPG];
#pragma unroll
    for (int i = 0; i < HPG; ++i) {
        const int h = min(h0 + i, a.heads - 1);
        xin[i] = *reinterpret_cast<const u32x4*>(a.src + row * a.src_rs + (int64_t)h * a.src_hs + 8 * c);
    }
    float wv[8];
    if (a.weight_kind == W_F32) {
        const f32x4 w0 = *reinterpret_cast<const f32x4*>(static_cast<const float*>(a.w) + 8 * c);
        const f32x4 w1 = *reinterpret_cast<const f32x4*>(static_cast<const float*>(a.w) + 8 * c + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) { wv[j] = w0[j]; wv[4 + j] = w1[j]; }
    } else if (a.weight_kind == W_BF16) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.w) + 8 * c);
#pragma unroll
        for (int j = 0; j < 4; ++j) { wv[2 * j] = lo_bf16(w[j]); wv[2 * j + 1] = hi_bf16(w[j]); }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) wv[j] = 1.0f;
    }
    const bool copy_row = row < a.n_copy;
    const int64_t toff = (copy_row ? 0 : row - a.n_copy) * a.tab_stride;
    const int P = a.rot >> 1;
    Rot2 rt[8];   // interleaved: pairs 4c..4c+3 in rt[0..3]; split-half: pairs of this lane's 8 dims
    if constexpr (KIND != TABLE_NONE) {
        if constexpr (PAIRING == PAIR_INTERLEAVED) {
#pragma unroll
            for (int j = 0; j < 4; ++j) rt[j] = rot_at<KIND>(a.ta, a.tb, toff, min(4 * c + j, P - 1));
        } else {
            const int hc = a.rot >> 4;   // chunks per half
            const int pc = c < hc ? c : c - hc;
#pragma unroll
            for (int j = 0; j < 8; ++j) rt[j] = rot_at<KIND>(a.ta, a.tb, toff, min(8 * pc + j, P - 1));
        }
    }

    // ---- per head: norm, rotation, store
#pragma unroll
    for (int i = 0; i < HPG; ++i) {
        const int h = h0 + i;
        uint16_t* dst = a.dst + row * a.dst_rs + (int64_t)min(h, a.heads - 1) * a.dst_hs + 8 * c;
        if (copy_row) {
            if (live && h < a.heads) *reinterpret_cast<u32x4*>(dst) = xin[i];
            continue;
        }
        float x[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x[2 * j] = lo_bf16(xin[i][j]);
            x[2 * j + 1] = hi_bf16(xin[i][j]);
        }
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) ss = fmaf(x[j], x[j], ss);
#pragma unroll
        for (int m = 1; m < 16; m <<= 1) ss += __shfl_xor(ss, m, 16);
        const float rr = rsqrtf(ss * (1.0f / D) + a.eps) * a.post_scale;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            x[j] = x[j] * rr * wv[j];
            if (a.round_norm) x[j] = (float)(bf16)x[j];
        }
        if constexpr (KIND != TABLE_NONE) {
            if constexpr (PAIRING == PAIR_INTERLEAVED) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const bool on = 8 * c + 2 * j < a.rot;
                    const float x0 = x[2 * j], x1 = x[2 * j + 1];
                    const float y0 = fmaf(rt[j].f00, x0, rt[j].f01 * x1);
                    const float y1 = fmaf(rt[j].f10, x0, rt[j].f11 * x1);
                    x[2 * j] = on ? y0 : x0;
                    x[2 * j + 1] = on ? y1 : x1;
                }
            } else {
                const int hc = a.rot >> 4;
                const int lane = threadIdx.x & 63, base = lane & ~15;
                const bool first = c < hc, second = c >= hc && c < 2 * hc;
                const int partner = base + (first ? c + hc : (second ? c - hc : c));
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float y = __shfl(x[j], partner, 64);
                    const float a0 = first ? x[j] : y, b0 = first ? y : x[j];   // (x_p, x_{p + rot/2})
                    const float ya = fmaf(rt[j].f00, a0, rt[j].f01 * b0);
                    const float yb = fmaf(rt[j].f10, a0, rt[j].f11 * b0);
                    x[j] = first ? ya : (second ? yb : x[j]);
                }
            }
        }
        if (live && h < a.heads) {
            u32x4 o;
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = pack_bf16x2(x[2 * j], x[2 * j + 1]);
            *reinterpret_cast<u32x4*>(dst) = o;
        }
    }
}

template <int KIND>
hipError_t launch_kind(const RopeArgs& a, unsigned blocks, hipStream_t stream) {
    if (a.pairing == PAIR_SPLIT_HALF)
        hipLaunchKernelGGL((rms_rope_kernel<KIND, PAIR_SPLIT_HALF>), dim3(blocks), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL((rms_rope_kernel<KIND, PAIR_INTERLEAVED>), dim3(blocks), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_rms_rope(const RopeArgs& a, hipStream_t stream) {
    const int64_t groups = a.rows * ((a.heads + HPG - 1) / HPG);
    const int64_t blocks = (groups + 15) / 16;
    if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidValue;
    switch (a.table_kind) {
        case TABLE_NONE: return launch_kind<TABLE_NONE>(a, (unsigned)blocks, stream);
        case TABLE_COSSIN_F32: return launch_kind<TABLE_COSSIN_F32>(a, (unsigned)blocks, stream);
        case TABLE_MAT2_BF16: return launch_kind<TABLE_MAT2_BF16>(a, (unsigned)blocks, stream);
        case TABLE_MAT2_F32: return launch_kind<TABLE_MAT2_F32>(a, (unsigned)blocks, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace lr
