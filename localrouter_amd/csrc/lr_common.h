// Shared device types and helpers for the gfx950 (CDNA4) joint-attention kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lr {

constexpr int D = 128;  // head dim: every kernel here is specialised for it

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));

// RoPE table kinds (per token row, per rotated pair p < rot/2)
enum TableKind : int {
    TABLE_NONE = 0,         // RMSNorm only
    TABLE_COSSIN_F32 = 1,   // cos fp32 [rows][stride] and sin fp32 [rows][stride] (Qwen-Image: [N, 64])
    TABLE_MAT2_BF16 = 2,    // bf16 [rows][stride] holding [rot/2][2][2] = {f00, f01, f10, f11} (MiniMax H3)
    TABLE_MAT2_F32 = 3,     // fp32, same layout as TABLE_MAT2_BF16
};
enum Pairing : int { PAIR_INTERLEAVED = 0, PAIR_SPLIT_HALF = 1 };
enum WeightKind : int { W_NONE = 0, W_F32 = 1, W_BF16 = 2 };

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
__device__ __forceinline__ float lo_bf16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Two floats -> packed bf16x2 bits (round to nearest even; v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 v;
    v[0] = (bf16)lo;
    v[1] = (bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
}

// The normalised value of H3's RMSNorm as the CPU restatement computes it -- fl32(fl64(fl64(x * rr) * w)), then
// rounded to bf16 (RNE) -- for a bf16 value x, a bf16 weight w and the row's factor rr in double. It is computed in
// fp32, y = (x * fl32(rr)) * w, which lies within 3.5 fp32 ulps of that fl32 value (three fp32 roundings against
// double ones). Unless y's low 16 bits lie within 8 ulps of a bf16 rounding tie (0x8000), both therefore round to the
// same bf16 value; near a tie (about 2^-12 of the values) the double computation itself decides, with an opaque step
// that keeps its two roundings (double -> fp32 -> bf16) from being folded into one double -> bf16 conversion.
// norm_bf16_exact8: the same for a lane's 8 values, with one (rarely taken) branch for the whole wave.
__device__ __forceinline__ float norm_bf16_slow(float x, double rr, float w) {
    // (the conversions are opaque so that the compiler computes them here, in the rare branch, and does not hoist
    // double copies of every x and w out of it)
    double xd, wd;
    asm volatile("v_cvt_f64_f32 %0, %1" : "=v"(xd) : "v"(x));
    asm volatile("v_cvt_f64_f32 %0, %1" : "=v"(wd) : "v"(w));
    float f = (float)(xd * rr * wd);
    asm volatile("" : "+v"(f));
    return (float)(bf16)f;
}
__device__ __forceinline__ bool near_bf16_tie(float y) { return (__float_as_uint(y) & 0xffffu) - (0x8000u - 8u) <= 16u; }
__device__ __forceinline__ float norm_bf16_exact(float x, double rr, float rr32, float w) {
    const float y = x * rr32 * w;
    return near_bf16_tie(y) ? norm_bf16_slow(x, rr, w) : (float)(bf16)y;
}
__device__ __forceinline__ void norm_bf16_exact8(float (&x)[8], double rr, const float (&w)[8]) {
    const float rr32 = (float)rr;
    float y[8];
    bool near = false;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        y[c] = x[c] * rr32 * w[c];
        near |= near_bf16_tie(y[c]);
    }
    if (__builtin_amdgcn_ballot_w64(near)) {
        // one value at a time: the double temporaries of eight would raise the register count of every caller
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            __builtin_amdgcn_sched_barrier(0);
            y[c] = near_bf16_tie(y[c]) ? norm_bf16_slow(x[c], rr, w[c]) : y[c];
        }
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) x[c] = (float)(bf16)y[c];
}

// Rotation coefficients of pair p at table row `row`: y_a = f00 x_a + f01 x_b, y_b = f10 x_a + f11 x_b.
struct Rot2 {
    float f00, f01, f10, f11;
};

__device__ __forceinline__ Rot2 load_rot(int kind, const void* ta, const void* tb, int64_t row_off, int p) {
    Rot2 r;
    if (kind == TABLE_COSSIN_F32) {
        const float c = static_cast<const float*>(ta)[row_off + p];
        const float s = static_cast<const float*>(tb)[row_off + p];
        r.f00 = c; r.f01 = -s; r.f10 = s; r.f11 = c;
    } else if (kind == TABLE_MAT2_BF16) {
        const u32x2 m = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(ta) + row_off + 4 * p);
        r.f00 = lo_bf16(m[0]); r.f01 = hi_bf16(m[0]); r.f10 = lo_bf16(m[1]); r.f11 = hi_bf16(m[1]);
    } else {
        const f32x4 m = *reinterpret_cast<const f32x4*>(static_cast<const float*>(ta) + row_off + 4 * p);
        r.f00 = m[0]; r.f01 = m[1]; r.f10 = m[2]; r.f11 = m[3];
    }
    return r;
}

}  // namespace lr
