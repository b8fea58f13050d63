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
