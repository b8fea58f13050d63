// Keys of the joint attention into the tile-image layout (tile_image.h): RMSNorm + RoPE of every key row j >= n_pre
// (table row j - n_pre; rows j < n_pre are an already normalised and rotated prefix and are copied). The values stay
// rows: the attention kernel reads the caller's value rows; the stage calls (copy_v) copy them into the workspace so
// that it holds everything a later call needs. The math per key row is the rms_rope kernel's (rms_rope.hip): the reference's
// kernels/cuda/minimax/kitchen/rms_rope.cu:37-230 / the Qwen-Image form of src/engines/qwen_image/triton_k.zig:44-53
// (fp32 weight, cos/sin fp32 tables), as wired by src/engines/qwen_image/dit.zig:252-263 (k via rms_rope into the
// key buffer after the prefix, v copied).
//
// One workgroup per (kv head, 64-key tile): it loads the tile's 64 key rows (256 contiguous bytes each), normalises
// and rotates them in registers, writes the image into LDS (a staging copy, see stg), then stores the 16 KB with fully
// coalesced 16-byte stores (copy_v: the 64 value rows too, 16 bytes a thread at a time). HBM-bound: 16 KB in and 16 KB
// out per tile (32 KB each with copy_v).
#include "lr_common.h"
#include "lr_kernels.h"
#include "tile_image.h"

namespace lr {

namespace {

#include "rope_rows.inc"

constexpr int KROWS = 4;   // key rows per thread (rows g, g + 16, g + 32, g + 48 of the tile)

// Where the 16 bytes at image offset o sit in the LDS staging copy: o with its 16-byte position inside the 128-byte
// line XORed by bits of the line index (a bijection on 16-byte units that keeps every line in place). The eight
// lanes of a write group put one key row's chunks 512-1024 bytes apart, all at the same position of their lines
// (eight lanes on four banks each: an 8-way conflict); the XOR spreads them over the line (conflict-free), while the
// copy-out, eight consecutive 16-byte units of one line per group, stays conflict-free.
__device__ __forceinline__ int stg(int o) { return o ^ ((((o >> 7) ^ (o >> 10)) & 7) << 4); }

// One 256-thread block: tile tile_id (kv head * tiles + tile) of the keys (and, copy_v, of the values), through img
// (16 KB of LDS: the key image).
template <int KIND, int PAIRING>
__device__ __forceinline__ void kv_tile_block(const KvImageArgs& a, int64_t tile_id, uint8_t* img) {
    const int tid = threadIdx.x, c = tid & 15, g = tid >> 4;
    if (tile_id == 0 && a.cnt)                         // the attention kernel's counters start each call at zero
        for (int x = tid; x < a.ncnt; x += 256) a.cnt[x] = 0;
    const int hk = (int)(tile_id / a.tiles), t = (int)(tile_id - (int64_t)hk * a.tiles);
    const int key0 = t * IMG_TILE_KEYS;

    // ---- the loads first: 4 key rows (16 bytes each), the weight, the first key row's table entries (the next row's
    // are loaded while a row is computed: two rows of entries live at a time)
    u32x4 xin[KROWS];
#pragma unroll
    for (int i = 0; i < KROWS; ++i) {
        const int key = min(key0 + g + 16 * i, a.Sk - 1);
        xin[i] = *reinterpret_cast<const u32x4*>(a.k + (int64_t)key * a.k_rs + (int64_t)hk * D + 8 * c);
    }
    // ---- values (copy_v): the tile's rows g + 16 i, dims 8 c .. +7, into the workspace's value rows
    // [tiles * 64][HK][128], zero past Sk; loaded and stored here, so that they hold no registers through the keys
    if (a.copy_v) {
        u32x4 vin[KROWS];
#pragma unroll
        for (int i = 0; i < KROWS; ++i) {
            const int key = key0 + g + 16 * i;
            vin[i] = key < a.Sk ? *reinterpret_cast<const u32x4*>(a.v + (int64_t)key * a.v_rs + (int64_t)hk * D + 8 * c)
                                : u32x4{0, 0, 0, 0};
        }
        uint16_t* vdst = static_cast<uint16_t*>(a.img_v) + (int64_t)hk * D + 8 * c;
#pragma unroll
        for (int i = 0; i < KROWS; ++i)
            *reinterpret_cast<u32x4*>(vdst + ((int64_t)(key0 + g + 16 * i) * a.HK) * D) = vin[i];
    }
    float wv[8];
    if (a.w) {
        const f32x4 w0 = *reinterpret_cast<const f32x4*>(a.w + 8 * c);
        const f32x4 w1 = *reinterpret_cast<const f32x4*>(a.w + 8 * c + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) { wv[j] = w0[j]; wv[4 + j] = w1[j]; }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) wv[j] = 1.0f;
    }
    const int P = a.rot >> 1;
    const int hc = a.rot >> 4;                           // split-half: 16-byte chunks per half
    // table entries of key row i in rt[i & 1]: interleaved, pairs 4c..4c+3 in [0..3]; split-half, the pairs of this
    // lane's 8 dims
    Rot2 rt[2][8];
    auto load_rt = [&](int i) __attribute__((always_inline)) {
        if constexpr (KIND != TABLE_NONE) {
            const int key = key0 + g + 16 * i;
            const int64_t toff = (int64_t)max(min(key, a.Sk - 1) - a.n_pre, 0) * a.tab_stride;
            if constexpr (PAIRING == PAIR_INTERLEAVED) {
                rot4<KIND>(a.ta, a.tb, toff, 4 * c, P, a.tab_vec, rt[i & 1]);
            } else {
                const int pc = c < hc ? c : c - hc;
                rot4<KIND>(a.ta, a.tb, toff, 8 * pc, P, a.tab_vec, rt[i & 1]);
                rot4<KIND>(a.ta, a.tb, toff, 8 * pc + 4, P, a.tab_vec, rt[i & 1] + 4);
            }
        }
    };
    load_rt(0);

    // ---- keys: norm, rotation, into the LDS image
#pragma unroll
    for (int i = 0; i < KROWS; ++i) {
        if (i + 1 < KROWS) load_rt(i + 1);
        __builtin_amdgcn_sched_barrier(0);   // row i + 1's entries in flight while row i is computed, no earlier
        const int r = g + 16 * i, key = key0 + r;
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
        const float rr = rsqrtf(ss * (1.0f / D) + a.eps);
        const bool copy = key < a.n_pre;
        float y[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] = x[j] * rr * wv[j];
        if constexpr (KIND != TABLE_NONE) {
            if constexpr (PAIRING == PAIR_INTERLEAVED) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const bool on = 8 * c + 2 * j < a.rot;
                    const float x0 = y[2 * j], x1 = y[2 * j + 1];
                    const float y0 = fmaf(rt[i & 1][j].f00, x0, rt[i & 1][j].f01 * x1);
                    const float y1 = fmaf(rt[i & 1][j].f10, x0, rt[i & 1][j].f11 * x1);
                    y[2 * j] = on ? y0 : x0;
                    y[2 * j + 1] = on ? y1 : x1;
                }
            } else {
                const int lane = tid & 63, base = lane & ~15;
                const bool first = c < hc, second = c >= hc && c < 2 * hc;
                const int partner = base + (first ? c + hc : (second ? c - hc : c));
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float o = __shfl(y[j], partner, 64);
                    const float a0 = first ? y[j] : o, b0 = first ? o : y[j];   // (x_p, x_{p + rot/2})
                    const float ya = fmaf(rt[i & 1][j].f00, a0, rt[i & 1][j].f01 * b0);
                    const float yb = fmaf(rt[i & 1][j].f10, a0, rt[i & 1][j].f11 * b0);
                    y[j] = first ? ya : (second ? yb : y[j]);
                }
            }
        }
        u32x4 o;
        if (key >= a.Sk) {
            o = u32x4{0, 0, 0, 0};
        } else if (copy) {
            o = xin[i];
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = pack_bf16x2(y[2 * j], y[2 * j + 1]);
        }
        *reinterpret_cast<u32x4*>(img + stg(img_k_offset(r, c))) = o;
    }
    __syncthreads();

    // ---- the key image out, 16 contiguous bytes per thread per pass
    uint8_t* kdst = reinterpret_cast<uint8_t*>(a.img_k) + tile_id * IMG_TILE_BYTES;
#pragma unroll
    for (int p = 0; p < IMG_TILE_BYTES / 4096; ++p) {
        const int off = p * 4096 + 16 * tid;
        *reinterpret_cast<u32x4*>(kdst + off) = *reinterpret_cast<const u32x4*>(img + stg(off));
    }
}

template <int KIND, int PAIRING>
__global__ __launch_bounds__(256) void kv_image_kernel(KvImageArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t img[IMG_TILE_BYTES];   // the key image
    kv_tile_block<KIND, PAIRING>(a, blockIdx.x, img);
}

// The joint attention's whole preparation in one launch: blocks [0, nkv) are key tiles (and value rows), the rest query rows
// (rope_rows_block over q: normalised and rotated into the prepared-query rows).
template <int KIND, int PAIRING>
__global__ __launch_bounds__(256) void joint_prep_kernel(KvImageArgs kv, RopeArgs q, int64_t nkv) {
    __shared__ __attribute__((aligned(16))) uint8_t img[IMG_TILE_BYTES];
    if ((int64_t)blockIdx.x < nkv) kv_tile_block<KIND, PAIRING>(kv, blockIdx.x, img);
    else rope_rows_block<KIND, PAIRING>(q, (int64_t)blockIdx.x - nkv);
}

template <int KIND>
hipError_t launch_kind(const KvImageArgs& a, hipStream_t stream) {
    const unsigned blocks = (unsigned)(a.tiles * a.HK);
    if (a.pairing == PAIR_SPLIT_HALF)
        hipLaunchKernelGGL((kv_image_kernel<KIND, PAIR_SPLIT_HALF>), dim3(blocks), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL((kv_image_kernel<KIND, PAIR_INTERLEAVED>), dim3(blocks), dim3(256), 0, stream, a);
    return hipGetLastError();
}

template <int KIND>
hipError_t launch_prep_kind(const KvImageArgs& kv, const RopeArgs& q, hipStream_t stream) {
    const int64_t nkv = kv.tiles * kv.HK;
    const int64_t nq = (q.rows * ((q.heads + 3) / 4) + 15) / 16;   // rope_rows_block: 16 groups of (row, 4 heads)
    if (nkv + nq > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 grid((unsigned)(nkv + nq));
    if (kv.pairing == PAIR_SPLIT_HALF)
        hipLaunchKernelGGL((joint_prep_kernel<KIND, PAIR_SPLIT_HALF>), grid, dim3(256), 0, stream, kv, q, nkv);
    else
        hipLaunchKernelGGL((joint_prep_kernel<KIND, PAIR_INTERLEAVED>), grid, dim3(256), 0, stream, kv, q, nkv);
    return hipGetLastError();
}

bool kv_args_ok(const KvImageArgs& a) {
    return a.Sk >= 1 && a.HK >= 1 && a.tiles == img_tiles(a.Sk) && (int64_t)a.tiles * a.HK <= 0x7fffffff;
}

}  // namespace

hipError_t launch_kv_image(const KvImageArgs& a, hipStream_t stream) {
    if (!kv_args_ok(a)) return hipErrorInvalidValue;
    switch (a.table_kind) {
        case TABLE_NONE: return launch_kind<TABLE_NONE>(a, stream);
        case TABLE_COSSIN_F32: return launch_kind<TABLE_COSSIN_F32>(a, stream);
        case TABLE_MAT2_BF16: return launch_kind<TABLE_MAT2_BF16>(a, stream);
        case TABLE_MAT2_F32: return launch_kind<TABLE_MAT2_F32>(a, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_joint_prep(const KvImageArgs& kv, const RopeArgs& q, hipStream_t stream) {
    // one table kind and pairing for both (the fused call's); the query blocks use q.table_kind's instantiation
    if (!kv_args_ok(kv) || q.rows < 1 || q.heads < 1 || q.table_kind != kv.table_kind || q.pairing != kv.pairing)
        return hipErrorInvalidValue;
    switch (kv.table_kind) {
        case TABLE_NONE: return launch_prep_kind<TABLE_NONE>(kv, q, stream);
        case TABLE_COSSIN_F32: return launch_prep_kind<TABLE_COSSIN_F32>(kv, q, stream);
        case TABLE_MAT2_BF16: return launch_prep_kind<TABLE_MAT2_BF16>(kv, q, stream);
        case TABLE_MAT2_F32: return launch_prep_kind<TABLE_MAT2_F32>(kv, q, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace lr
