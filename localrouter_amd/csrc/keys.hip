// Key compaction for attention under a key-padding mask (Kandinsky-6's attention.Call with mask = .keys,
// src/engines/kandinsky6/dit/attention.zig:21-27: a u8 per key, nonzero = keep; SDPA's additive 0 / -inf mask). The
// kept keys and their value rows are gathered, in order, into a workspace, and the attention runs over them:
// softmax over the kept keys equals softmax over all keys with the others at -inf.
//
// compact_scan_kernel: one workgroup. Thread i counts the kept keys of its contiguous chunk, an exclusive scan over
// the workgroup gives each chunk its first output slot, and idx[slot] = key for every kept key (slots < n_valid).
// gather_rows_kernel: one 16-byte chunk of a K row and of a V row per thread, for rows j < n_valid.
#include "lr_common.h"
#include "lr_kernels.h"

namespace lr {
namespace {

constexpr int SCAN_THREADS = 1024;

__global__ __launch_bounds__(SCAN_THREADS) void compact_scan_kernel(const uint8_t* kmask, int nkeys, int n_valid,
                                                                    int* idx) {
    __shared__ int part[SCAN_THREADS];
    const int t = threadIdx.x;
    const int per = (nkeys + SCAN_THREADS - 1) / SCAN_THREADS;
    const int b = t * per, e = min(nkeys, b + per);
    int cnt = 0;
    for (int j = b; j < e; ++j) cnt += kmask[j] != 0;
    part[t] = cnt;
    __syncthreads();
    // Hillis-Steele inclusive scan over the workgroup
    for (int off = 1; off < SCAN_THREADS; off <<= 1) {
        const int add = t >= off ? part[t - off] : 0;
        __syncthreads();
        part[t] += add;
        __syncthreads();
    }
    int slot = part[t] - cnt;
    for (int j = b; j < e; ++j)
        if (kmask[j] != 0) {
            if (slot < n_valid) idx[slot] = j;
            ++slot;
        }
}

// A slot whose index is not a key (the mask holds fewer kept keys than n_valid: a caller error) gets zero rows
// rather than a read out of bounds.
__global__ void gather_rows_kernel(const uint16_t* k, const uint16_t* v, int64_t kv_rs, const int* idx, int nkeys,
                                   int n_valid, int row_chunks, uint16_t* kc, uint16_t* vc) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)n_valid * row_chunks) return;
    const int j = (int)(i / row_chunks), c = (int)(i - (int64_t)j * row_chunks);
    const int r = idx[j];
    const int64_t dst = (int64_t)j * row_chunks * 8 + 8 * c;
    u32x4 kk = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
    if ((unsigned)r < (unsigned)nkeys) {
        const int64_t src = (int64_t)r * kv_rs + 8 * c;
        kk = *reinterpret_cast<const u32x4*>(k + src);
        vv = *reinterpret_cast<const u32x4*>(v + src);
    }
    *reinterpret_cast<u32x4*>(kc + dst) = kk;
    *reinterpret_cast<u32x4*>(vc + dst) = vv;
}

}  // namespace

hipError_t launch_compact_keys(const void* k, const void* v, int64_t kv_rs, const uint8_t* kmask, int nkeys,
                               int n_valid, int HK, void* idx, void* kc, void* vc, hipStream_t stream) {
    hipLaunchKernelGGL(compact_scan_kernel, dim3(1), dim3(SCAN_THREADS), 0, stream, kmask, nkeys, n_valid,
                       static_cast<int*>(idx));
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int row_chunks = HK * D / 8;
    const int64_t n = (int64_t)n_valid * row_chunks;
    hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v), kv_rs,
                       static_cast<const int*>(idx), nkeys, n_valid, row_chunks, static_cast<uint16_t*>(kc),
                       static_cast<uint16_t*>(vc));
    return hipGetLastError();
}

}  // namespace lr
