/* Host-side RoPE position and table builders for the joint-attention path: plain C ABI, CPU only.
 *
 * The engines build these tables once per shape on the host and upload them (the cos/sin tables that
 * lr_rms_rope_bf16 / lr_joint_attention_fused read as LR_TABLE_COSSIN_F32, and MiniMax H3's [S, 48, 2, 2] bf16 table
 * that lr_rms_rope_qk_bf16 reads). Every function writes caller-owned host buffers, allocates nothing and touches no
 * GPU. Functions that can fail return 0 on success and 1 (the library's hipErrorInvalidValue convention) when an
 * argument is rejected, before anything is written.
 *
 * Qwen-Image: ids [N, 3] f32 = (frame or position, row, column); 64 frequencies over axes of 16 / 56 / 56 dims;
 * angle = f64(id) * omega in f64, cos and sin in f64 rounded to f32; tables [N, 64] f32, interleaved pairs.
 * MiniMax H3: positions [S, 3] f64 (t, h, w) of the packed [text | cond | audio | video] layout; angle =
 * f32(pos) * inv_freq[j] in f32, cos and sin in f64 rounded to f32 then to bf16 (nearest even); table entry
 * (r, 16 axis + j) = [c, -s, s, c] bf16 bits.
 * The synthetic BASELINE shapes (2D image grid, three-frame edit layout, 3D video grid) are this build's own
 * definitions: text tokens first and un-rotated (cos 1, sin 0).
 */
#ifndef LR_ROPE_H
#define LR_ROPE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The 64 Qwen-Image frequencies as the engine loads them (kernels/qwen_image/rope_omega.json, read by smath.omegas,
 * src/engines/qwen_image/smath.zig:112-126), f64 into out[64]. */
/* The engines' portable sin and cos of n f64 angles (src/engines/qwen_image/smath.zig:18-52: Cody-Waite reduction by
 * pi/2 in three parts, fdlibm's kernel polynomials, the same operations in the same order), which every table below
 * uses. Returns 0, or 1 for a bad argument. */
int lr_rope_sincos(const double* x, int64_t n, double* sin_out, double* cos_out);

void lr_rope_qwen_omegas(double* out);

/* Text ids: position first + i on all three axes (src/engines/qwen_image/rope.zig:11-13). ids [n, 3] f32. */
int lr_rope_qwen_text_ids(float* ids, int n, int first);

/* Image ids of an h x w latent at frame `pos`, rows and columns centred, half-pixel shifted for odd sides against
 * the target's parity (rope.zig:16-28). ids [h * w, 3] f32, row-major grid. */
int lr_rope_qwen_image_ids(float* ids, int h, int w, int pos, int target_h, int target_w);

/* cos, sin [n, 64] f32 from ids [n, 3] (rope.zig:31-45). omegas: 64 values, or NULL for the engine's. */
int lr_rope_qwen_table(const float* ids, int n, const double* omegas, float* cos_out, float* sin_out);

/* The 2D grid table of the BASELINE image shapes: n_text un-rotated rows, then gh x gw tokens; pairs 0-31 rotate by
 * the row, pairs 32-63 by the column, omega_j = theta^(-2j/64). cos, sin [n_text + gh * gw, 64] f32. */
int lr_rope_grid2d_table(int n_text, int gh, int gw, double theta, float* cos_out, float* sin_out);

/* The edit layout: n_text un-rotated rows, then `frames` gh x gw latents, latent f on frame f, ids as
 * lr_rope_qwen_image_ids, the engine's frequencies. cos, sin [n_text + frames * gh * gw, 64] f32. */
int lr_rope_edit_table(int n_text, int frames, int gh, int gw, float* cos_out, float* sin_out);

/* The video layout: n_text un-rotated rows, then t x gh x gw tokens (frame-major); t/h/w take 32/48/48 dims
 * (16/24/24 pairs), omega_{a,j} = theta^(-2j/d_a), integer positions. cos, sin [n_text + t * gh * gw, 64] f32. */
int lr_rope_video3d_table(int n_text, int t, int gh, int gw, double theta, float* cos_out, float* sin_out);

/* Rows of the H3 packed layout: l + (first_frame ? (h/2)(w/2) : 0) + 2 a + t (h/2)(w/2); -1 for a bad argument
 * (src/engines/minimax_h3/layout.zig:85-115). */
int64_t lr_rope_h3_rows(int l, int t, int h, int w, int a, int first_frame);

/* H3 positions [rows, 3] f64 (layout.zig:85-115). */
int lr_rope_h3_positions(int l, int t, int h, int w, int a, int first_frame, double* pos);

/* H3 table [rows, 48, 2, 2] bf16 bits from positions [rows, 3] and 16 f32 inverse frequencies
 * (layout.zig:117-134). */
int lr_rope_h3_table(const double* pos, int64_t rows, const float* inv_freq, uint16_t* out);

#ifdef __cplusplus
}
#endif

#endif /* LR_ROPE_H */
