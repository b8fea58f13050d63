// Host RoPE position and table builders (C ABI of include/lr_rope.h): CPU code, no GPU calls, no allocation.
//
// Qwen-Image: src/engines/qwen_image/rope.zig:7-45 (ids and cos/sin tables), frequencies of
// kernels/qwen_image/rope_omega.json as smath.omegas reads them (smath.zig:112-126). MiniMax H3:
// src/engines/minimax_h3/layout.zig:60-134 (packed-layout positions, the [S, 48, 2, 2] bf16 table). The reference
// computes sin/cos with its own portable f64 routine (smath.zig:18-52), and so does this file (engine_sincos below),
// so that the tables are the engine's bits, not libm's.
#include <cmath>
#include <cstdint>
#include <cstring>

#include "../../include/lr_rope.h"

namespace {

constexpr int kPairs = 64;

// The 64 engine frequencies, axis by axis (16 / 56 / 56 dims), as f64 bit patterns: torch's float64
// 1 / 10000 ** linspace(0, (d - 2) / d, d / 2) per axis, frozen in the reference's rope_omega.json.
constexpr uint64_t kQwenOmegaBits[kPairs] = {
    0x3ff0000000000000ull, 0x3fd43d136248490full, 0x3fb999999999999aull, 0x3fa030dc4ea03a72ull,
    0x3f847ae147ae147bull, 0x3f69e7c6e43390b6ull, 0x3f50624dd2f1a9fcull, 0x3f34b96be9c2da2cull,
    0x3ff0000000000000ull, 0x3fe707aa3f9e1202ull, 0x3fe093069178d379ull, 0x3fd7db4a2009c6e3ull,
    0x3fd12b542ba56564ull, 0x3fc8b682a4336478ull, 0x3fc1c9194d504805ull, 0x3fb999999999999aull,
    0x3fb26c8832e4db35ull, 0x3faa84d74f27b8c3ull, 0x3fa315d4e66e38b8ull, 0x3f9b7886ac3bd56dull,
    0x3f93c53550291d2dull, 0x3f8c74f54880733dull, 0x3f847ae147ae147bull, 0x3f7d7a7384a15eb3ull,
    0x3f753712a5b96096ull, 0x3f6e8954a3e38deaull, 0x3f65fa0556964454ull, 0x3f5fa1eee6a82eaaull,
    0x3f56c3f76d338f61ull, 0x3f50624dd2f1a9fcull, 0x3f47952936e77efcull, 0x3f40f8dbb7c7807dull,
    0x3f386ddd4fe93e54ull, 0x3f3194d11211d043ull, 0x3f294e58b8868bbbull, 0x3f22365f8a8fa5e7ull,
    0x3ff0000000000000ull, 0x3fe707aa3f9e1202ull, 0x3fe093069178d379ull, 0x3fd7db4a2009c6e3ull,
    0x3fd12b542ba56564ull, 0x3fc8b682a4336478ull, 0x3fc1c9194d504805ull, 0x3fb999999999999aull,
    0x3fb26c8832e4db35ull, 0x3faa84d74f27b8c3ull, 0x3fa315d4e66e38b8ull, 0x3f9b7886ac3bd56dull,
    0x3f93c53550291d2dull, 0x3f8c74f54880733dull, 0x3f847ae147ae147bull, 0x3f7d7a7384a15eb3ull,
    0x3f753712a5b96096ull, 0x3f6e8954a3e38deaull, 0x3f65fa0556964454ull, 0x3f5fa1eee6a82eaaull,
    0x3f56c3f76d338f61ull, 0x3f50624dd2f1a9fcull, 0x3f47952936e77efcull, 0x3f40f8dbb7c7807dull,
    0x3f386ddd4fe93e54ull, 0x3f3194d11211d043ull, 0x3f294e58b8868bbbull, 0x3f22365f8a8fa5e7ull,
};
constexpr int kQwenAxes[3] = {16, 56, 56};

double bits_to_f64(uint64_t b) {
    double d;
    std::memcpy(&d, &b, sizeof d);
    return d;
}

uint32_t f32_bits(float f) {
    uint32_t b;
    std::memcpy(&b, &f, sizeof b);
    return b;
}

// round to nearest even, finite inputs (layout.zig:31-34)
uint16_t f32_to_bf16(float f) {
    const uint64_t b = f32_bits(f);
    return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

// The engine's portable sin / cos of an f64 angle (smath.zig:18-52): Cody-Waite reduction by pi/2 with pi/2 split
// in three parts (the first 33 bits exact in n * pio2_1 for |n| < 2^20), then the polynomial kernels of fdlibm
// (Sun Microsystems, 1993: k_sin.c, k_cos.c, the reduction constants of e_rem_pio2.c), and the quadrant n mod 4.
// The operation order fixes the bits; this file is compiled without FMA contraction.
constexpr double kInvPio2 = 6.36619772367581382433e-01;
constexpr double kPio2_1 = 1.57079632673412561417e+00;
constexpr double kPio2_2 = 6.07710050630396597660e-11;
constexpr double kPio2_3 = 2.02226624871116645580e-21;
constexpr double kS[6] = {-1.66666666666666324348e-01, 8.33333333332248946124e-03, -1.98412698298579493134e-04,
                          2.75573137070700676789e-06, -2.50507602534068634195e-08, 1.58969099521155010221e-10};
constexpr double kC[6] = {4.16666666666666019037e-02, -1.38888888888741095749e-03, 2.48015872894767294178e-05,
                          -2.75573143513906633035e-07, 2.08757232129817482790e-09, -1.13596475577881948265e-11};

void engine_sincos(double x, double* sin_out, double* cos_out) {
    const double fn = std::floor(x * kInvPio2 + 0.5);
    const int64_t n = (int64_t)fn;
    const double r = ((x - fn * kPio2_1) - fn * kPio2_2) - fn * kPio2_3;
    const double z = r * r;
    // kernel sin: r + r^3 (s1 + z (s2 + z (s3 + z (s4 + z (s5 + z s6)))))
    const double v = z * r;
    const double sr = kS[1] + z * (kS[2] + z * (kS[3] + z * (kS[4] + z * kS[5])));
    const double sv = r + v * (kS[0] + z * sr);
    // kernel cos: 1 - z/2 + z^2 (c1 + ...), the 1 - z/2 part with its rounding error carried
    const double cr = z * (kC[0] + z * (kC[1] + z * (kC[2] + z * (kC[3] + z * (kC[4] + z * kC[5])))));
    const double hz = 0.5 * z;
    const double w = 1.0 - hz;
    const double cv = w + (((1.0 - w) - hz) + z * cr);
    switch ((uint64_t)n & 3u) {
        case 0: *sin_out = sv; *cos_out = cv; break;
        case 1: *sin_out = cv; *cos_out = -sv; break;
        case 2: *sin_out = -sv; *cos_out = -cv; break;
        default: *sin_out = -cv; *cos_out = sv; break;
    }
}

// omega_j = 1 / theta^(2j/d), j < d/2
double axis_omega(int d, int j, double theta) { return 1.0 / std::pow(theta, 2.0 * (double)j / (double)d); }

void identity_rows(int64_t n, float* c, float* s) {
    for (int64_t i = 0; i < n * kPairs; ++i) {
        c[i] = 1.0f;
        s[i] = 0.0f;
    }
}

// one table row: angle = pos[axis of pair p] * om[p] in f64
void table_row(const double* pos3, const int* axis_of_pair, const double* om, float* c, float* s) {
    for (int p = 0; p < kPairs; ++p) {
        const double ang = pos3[axis_of_pair[p]] * om[p];
        double sv, cv;
        engine_sincos(ang, &sv, &cv);
        c[p] = (float)cv;
        s[p] = (float)sv;
    }
}

// pair -> axis for axes of d0 / d1 / d2 dims (d0 + d1 + d2 = 128)
void pair_axes(const int* dims, int* axis_of_pair) {
    int p = 0;
    for (int ax = 0; ax < 3; ++ax)
        for (int j = 0; j < dims[ax] / 2; ++j) axis_of_pair[p++] = ax;
}

// H3 per-axis position (layout.zig:78-82): (i * (ratio / n) + (1 - ratio) / 2) * 32, ratio = dim / area, n = dim / 2
double h3_axis(int dim, double area, int64_t i) {
    const double ratio = (double)dim / area;
    const double n = (double)(dim / 2);
    return ((double)i * (ratio / n) + (1.0 - ratio) / 2.0) * 32.0;
}

constexpr double kH3FramePerToken[5] = {1.0, 4.0, 4.0, 4.0, 4.0};   // layout.zig:12
constexpr double kH3FrameRescale = 5.0 / 3.0;                        // layout.zig:13

}  // namespace

extern "C" {

int lr_rope_sincos(const double* x, int64_t n, double* sin_out, double* cos_out) {
    if (n < 0 || (n > 0 && (!x || !sin_out || !cos_out))) return 1;
    for (int64_t i = 0; i < n; ++i) engine_sincos(x[i], sin_out + i, cos_out + i);
    return 0;
}

void lr_rope_qwen_omegas(double* out) {
    for (int p = 0; p < kPairs; ++p) out[p] = bits_to_f64(kQwenOmegaBits[p]);
}

int lr_rope_qwen_text_ids(float* ids, int n, int first) {
    if (n < 0 || !ids) return 1;
    for (int i = 0; i < n; ++i) ids[3 * i] = ids[3 * i + 1] = ids[3 * i + 2] = (float)(first + i);
    return 0;
}

int lr_rope_qwen_image_ids(float* ids, int h, int w, int pos, int target_h, int target_w) {
    if (h <= 0 || w <= 0 || target_h <= 0 || target_w <= 0 || !ids) return 1;
    // f32 arithmetic throughout, as the engine's
    const float fh = (float)h, fw = (float)w;
    const float sh = -(fh - (float)(h / 2)) + 0.5f * ((float)(h % 2) - (float)(target_h % 2));
    const float sw = -(fw - (float)(w / 2)) + 0.5f * ((float)(w % 2) - (float)(target_w % 2));
    for (int y = 0; y < h; ++y)
        for (int x = 0; x < w; ++x) {
            float* r = ids + 3 * ((int64_t)y * w + x);
            r[0] = (float)pos;
            r[1] = (float)y + sh;
            r[2] = (float)x + sw;
        }
    return 0;
}

int lr_rope_qwen_table(const float* ids, int n, const double* omegas, float* cos_out, float* sin_out) {
    if (n < 0 || !ids || !cos_out || !sin_out) return 1;
    double om[kPairs];
    if (omegas) std::memcpy(om, omegas, sizeof om);
    else lr_rope_qwen_omegas(om);
    int axis_of_pair[kPairs];
    pair_axes(kQwenAxes, axis_of_pair);
    for (int i = 0; i < n; ++i) {
        const double pos3[3] = {(double)ids[3 * i], (double)ids[3 * i + 1], (double)ids[3 * i + 2]};
        table_row(pos3, axis_of_pair, om, cos_out + (int64_t)i * kPairs, sin_out + (int64_t)i * kPairs);
    }
    return 0;
}

int lr_rope_grid2d_table(int n_text, int gh, int gw, double theta, float* cos_out, float* sin_out) {
    if (n_text < 0 || gh < 0 || gw < 0 || !(theta > 0.0) || !cos_out || !sin_out) return 1;
    identity_rows(n_text, cos_out, sin_out);
    double om[kPairs];
    int axis_of_pair[kPairs];
    for (int p = 0; p < kPairs; ++p) {
        om[p] = axis_omega(64, p % 32, theta);
        axis_of_pair[p] = p < 32 ? 0 : 1;
    }
    for (int r = 0; r < gh; ++r)
        for (int c = 0; c < gw; ++c) {
            const int64_t row = n_text + (int64_t)r * gw + c;
            const double pos[2] = {(double)r, (double)c};
            table_row(pos, axis_of_pair, om, cos_out + row * kPairs, sin_out + row * kPairs);
        }
    return 0;
}

int lr_rope_edit_table(int n_text, int frames, int gh, int gw, float* cos_out, float* sin_out) {
    if (n_text < 0 || frames < 0 || gh <= 0 || gw <= 0 || !cos_out || !sin_out) return 1;
    identity_rows(n_text, cos_out, sin_out);
    double om[kPairs];
    lr_rope_qwen_omegas(om);
    int axis_of_pair[kPairs];
    pair_axes(kQwenAxes, axis_of_pair);
    // the f32 ids of lr_rope_qwen_image_ids, widened to f64
    const float sh = -((float)gh - (float)(gh / 2));
    const float sw = -((float)gw - (float)(gw / 2));
    for (int f = 0; f < frames; ++f)
        for (int y = 0; y < gh; ++y)
            for (int x = 0; x < gw; ++x) {
                const int64_t row = n_text + ((int64_t)f * gh + y) * gw + x;
                const double pos3[3] = {(double)(float)f, (double)((float)y + sh), (double)((float)x + sw)};
                table_row(pos3, axis_of_pair, om, cos_out + row * kPairs, sin_out + row * kPairs);
            }
    return 0;
}

int lr_rope_video3d_table(int n_text, int t, int gh, int gw, double theta, float* cos_out, float* sin_out) {
    if (n_text < 0 || t < 0 || gh < 0 || gw < 0 || !(theta > 0.0) || !cos_out || !sin_out) return 1;
    identity_rows(n_text, cos_out, sin_out);
    const int dims[3] = {32, 48, 48};
    double om[kPairs];
    int axis_of_pair[kPairs];
    pair_axes(dims, axis_of_pair);
    for (int p = 0, ax = 0; ax < 3; ++ax)
        for (int j = 0; j < dims[ax] / 2; ++j) om[p++] = axis_omega(dims[ax], j, theta);
    for (int f = 0; f < t; ++f)
        for (int y = 0; y < gh; ++y)
            for (int x = 0; x < gw; ++x) {
                const int64_t row = n_text + ((int64_t)f * gh + y) * gw + x;
                const double pos3[3] = {(double)f, (double)y, (double)x};
                table_row(pos3, axis_of_pair, om, cos_out + row * kPairs, sin_out + row * kPairs);
            }
    return 0;
}

int64_t lr_rope_h3_rows(int l, int t, int h, int w, int a, int first_frame) {
    if (l < 0 || t < 0 || h < 2 || w < 2 || a < 0) return -1;
    const int64_t frame = (int64_t)(h / 2) * (w / 2);
    return (int64_t)l + (first_frame ? frame : 0) + 2 * (int64_t)a + (int64_t)t * frame;
}

int lr_rope_h3_positions(int l, int t, int h, int w, int a, int first_frame, double* pos) {
    if (lr_rope_h3_rows(l, t, h, w, a, first_frame) < 0 || !pos) return 1;
    const double area = std::sqrt((double)h * (double)w);
    const int fh = h / 2, fw = w / 2;
    const double w_lo = h3_axis(w, area, 0), w_hi = h3_axis(w, area, fw - 1);
    int64_t r = 0;
    auto put = [&](double a0, double a1, double a2) {
        pos[3 * r] = a0;
        pos[3 * r + 1] = a1;
        pos[3 * r + 2] = a2;
        ++r;
    };
    auto frame_at = [&](double tpos) {
        for (int y = 0; y < fh; ++y)
            for (int x = 0; x < fw; ++x) put(tpos, h3_axis(h, area, y), h3_axis(w, area, x));
    };
    for (int i = 0; i < l; ++i) put((double)i, 0.0, 0.0);                         // text
    const double cursor = (double)l;
    if (first_frame) frame_at(cursor);                                            // condition frame
    for (int ch = 0; ch < 2; ++ch)                                                // audio, two channels
        for (int i = 0; i < a; ++i) put(cursor + (double)i, 0.0, ch == 0 ? w_lo : w_hi);
    double cum = 0.0;
    for (int k = 0; k < t; ++k) {                                                 // video frames
        frame_at(cursor + cum);
        cum += kH3FrameRescale * kH3FramePerToken[k % 5];
    }
    return 0;
}

int lr_rope_h3_table(const double* pos, int64_t rows, const float* inv_freq, uint16_t* out) {
    if (rows < 0 || !pos || !inv_freq || !out) return 1;
    for (int64_t r = 0; r < rows; ++r)
        for (int ax = 0; ax < 3; ++ax) {
            const float p = (float)pos[3 * r + ax];
            for (int j = 0; j < 16; ++j) {
                const float ang = p * inv_freq[j];   // f32 product
                double sv, cv;
                engine_sincos((double)ang, &sv, &cv);
                const float c = (float)cv, s = (float)sv;
                uint16_t* e = out + (r * 48 + ax * 16 + j) * 4;
                e[0] = f32_to_bf16(c);
                e[1] = f32_to_bf16(-s);
                e[2] = f32_to_bf16(s);
                e[3] = f32_to_bf16(c);
            }
        }
    return 0;
}

}  // extern "C"
