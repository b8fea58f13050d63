// The "tile image" layout of prepared keys: every 64-key tile of a kv head is stored in HBM exactly as the attention
// kernel keeps it in LDS, as 16 operand fragments of 1 KB. A fragment is the operand of one
// v_mfma_f32_32x32x16_bf16 for all 64 lanes of a wave, lane l's 16 bytes at byte 16 l, so that
//   - one contiguous 1 KB global -> LDS load (16 bytes per lane) moves one fragment, and
//   - one ds_read_b128 at (fragment base + 16 l), the base an immediate offset, reads it back without bank conflicts.
//
// Keys (A operand of S^T = K Q^T, rows = keys, k = dims): fragment f = 8 mb + ks of a tile, lane l = 32 hf + n holds
// dims 16 ks + 8 hf .. +7 of key 32 mb + key_perm(n). key_perm swaps bits 2 and 3 of a row index, so that the 16
// score registers of a lane (32x32 MFMA output rows 8 g + 4 hf + r, g, r < 4) are the keys 16 (g >> 1) + 8 hf +
// 4 (g & 1) + r: registers 0-7 are keys 8 hf .. 8 hf + 7 of the block's first 16-key step, registers 8-15 those of its
// second -- exactly the B operand (P^T, 8 consecutive keys per lane) of the P V product, so P needs no shuffle.
//
// The values are not imaged: the attention kernel reads value rows and transposes them with its LDS reads
// (attn_stream.hip).
//
// Keys past the last key of a head are zero. Tile t of kv head g starts at byte (g * tiles + t) * 16384.
#pragma once
#include <stdint.h>

namespace lr {

constexpr int IMG_TILE_KEYS = 64;
constexpr int IMG_FRAG_BYTES = 1024;
constexpr int IMG_TILE_BYTES = 16 * IMG_FRAG_BYTES;

// the key whose row the 32x32 MFMA row m (0..31) holds: bits 2 and 3 swapped (an involution)
__host__ __device__ constexpr int img_key_perm(int m) { return (m & 0x13) | ((m & 4) << 1) | ((m & 8) >> 1); }

// byte offset, within a tile, of the 16 bytes holding dims 8 c .. 8 c + 7 (c < 16) of key r (r < 64)
__host__ __device__ constexpr int img_k_offset(int r, int c) {
    return (8 * (r >> 5) + (c >> 1)) * IMG_FRAG_BYTES + (32 * (c & 1) + img_key_perm(r & 31)) * 16;
}

inline int64_t img_tiles(int Sk) { return (Sk + IMG_TILE_KEYS - 1) / IMG_TILE_KEYS; }
// bytes of the key images of HK kv heads (and of the workspace's value area: tiles * 64 rows of HK * 256 bytes)
inline int64_t img_bytes(int Sk, int HK) { return img_tiles(Sk) * HK * IMG_TILE_BYTES; }

}  // namespace lr
