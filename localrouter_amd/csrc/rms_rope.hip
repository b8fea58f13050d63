// Per-(token, head) RMSNorm + RoPE over bf16 rows, for gfx950.
//
// Semantics: kernels/cuda/minimax/kitchen/rms_rope.cu:37-230 with rope_device.cuh:65-98 (MiniMax H3: rrms =
// 1/sqrt(sum(x^2)/128 + eps), y = x * rrms * w, the normalised value rounded to bf16 before the rotation, pairs
// (i, i + rot/2) rotated by [f00 f01; f10 f11] from a bf16 table [rows][rot/2][2][2], dims >= rot norm-only) and the
// Qwen-Image form launched by src/engines/qwen_image/triton_k.zig:44-53 (fp32 weight, fp32 cos/sin [N, rot/2]).
// Each (row, head) is one group of 16 lanes; lane c holds dims 8c..8c+7 as one 16-byte load, the sum of squares is a
// 4-step xor butterfly inside the group, and a split-half partner chunk comes from lane c +- rot/16 of the same group.
// HBM-bound by design: 256 bytes in and 256 bytes out per (row, head).
#include "lr_common.h"
#include "lr_kernels.h"

namespace lr {

namespace {

__global__ __launch_bounds__(256) void rms_rope_kernel(RopeArgs a) {
    const int tid = threadIdx.x;
    const int c = tid & 15;
    const int64_t g = (int64_t)blockIdx.x * 16 + (tid >> 4);   // (row, head) group
    const int64_t total = a.rows * a.heads;
    const bool live = g < total;
    const int64_t gg = live ? g : total - 1;                   // dead groups mirror the last one, then skip the store
    const int64_t row = gg / a.heads;
    const int head = (int)(gg - row * a.heads);
    const uint16_t* src = a.src + row * a.src_rs + (int64_t)head * a.src_hs + 8 * c;
    uint16_t* dst = a.dst + row * a.dst_rs + (int64_t)head * a.dst_hs + 8 * c;
    const u32x4 w = *reinterpret_cast<const u32x4*>(src);
    if (row < a.n_copy) {   // uniform within the group
        if (live) *reinterpret_cast<u32x4*>(dst) = w;
        return;
    }
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[2 * i] = lo_bf16(w[i]);
        x[2 * i + 1] = hi_bf16(w[i]);
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = fmaf(x[j], x[j], ss);
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) ss += __shfl_xor(ss, m, 16);
    const float rr = rsqrtf(ss * (1.0f / D) + a.eps);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int d = 8 * c + j;
        float wd = 1.0f;
        if (a.weight_kind == W_F32) wd = static_cast<const float*>(a.w)[d];
        else if (a.weight_kind == W_BF16) wd = bf16_bits_to_f32(static_cast<const uint16_t*>(a.w)[d]);
        x[j] = x[j] * rr * wd;
        if (a.round_norm) x[j] = (float)(bf16)x[j];
    }
    if (a.table_kind != TABLE_NONE) {
        const int64_t toff = (row - a.n_copy) * a.tab_stride;
        if (a.pairing == PAIR_INTERLEAVED) {
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                const int d = 8 * c + j;
                if (d < a.rot) {
                    const Rot2 r = load_rot(a.table_kind, a.ta, a.tb, toff, d >> 1);
                    const float x0 = x[j], x1 = x[j + 1];
                    x[j] = fmaf(r.f00, x0, r.f01 * x1);
                    x[j + 1] = fmaf(r.f10, x0, r.f11 * x1);
                }
            }
        } else {
            // rot % 16 == 0: chunk c < rot/16 holds first elements, chunk c + rot/16 their partners
            const int hc = a.rot >> 4;
            const int lane = threadIdx.x & 63, base = lane & ~15;
            const bool first = c < hc, second = c >= hc && c < 2 * hc;
            const int partner = base + (first ? c + hc : (second ? c - hc : c));
            float y[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) y[j] = __shfl(x[j], partner, 64);
            if (first || second) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int p = (first ? 8 * c : 8 * c - 8 * hc) + j;
                    const Rot2 r = load_rot(a.table_kind, a.ta, a.tb, toff, p);
                    if (first) x[j] = fmaf(r.f00, x[j], r.f01 * y[j]);
                    else x[j] = fmaf(r.f10, y[j], r.f11 * x[j]);
                }
            }
        }
    }
    if (live) {
        u32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
        *reinterpret_cast<u32x4*>(dst) = o;
    }
}

}  // namespace

hipError_t launch_rms_rope(const RopeArgs& a, hipStream_t stream) {
    const int64_t groups = a.rows * a.heads;
    const int64_t blocks = (groups + 15) / 16;
    if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rms_rope_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace lr
