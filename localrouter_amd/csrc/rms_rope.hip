// Per-(token, head) RMSNorm + RoPE over bf16 rows, for gfx950: the standalone pass (lr_rms_rope_bf16, the queries of
// lr_joint_q_prepare). The work of one block is rope_rows_block (rope_rows.inc).
// HBM-bound by design: 256 bytes in and 256 bytes out per (row, head).
#include "lr_common.h"
#include "lr_kernels.h"

namespace lr {

namespace {

#include "rope_rows.inc"

template <int KIND, int PAIRING>
__global__ __launch_bounds__(256) void rms_rope_kernel(RopeArgs a) {
    rope_rows_block<KIND, PAIRING>(a, blockIdx.x);
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
