// Deterministic exclusive scan of int32 counts (fixed order): one workgroup
// for short inputs, three passes otherwise.
#include "nlist.hpp"

namespace rune {

namespace {
constexpr int kScanBlock = 1024;

__device__ inline int32_t block_exclusive(int32_t v, int32_t *lds, int32_t *total) {
    const int t = threadIdx.x;
    lds[t] = v;
    __syncthreads();
    for (int off = 1; off < kScanBlock; off <<= 1) {
        int32_t add = (t >= off) ? lds[t - off] : 0;
        __syncthreads();
        lds[t] += add;
        __syncthreads();
    }
    int32_t incl = lds[t];
    if (total && t == kScanBlock - 1) *total = incl;
    return incl - v;
}

__global__ void __launch_bounds__(kScanBlock) scan_blocks(const int32_t *in, int32_t *out,
                                                          int64_t n, int32_t *block_sums) {
    __shared__ int32_t lds[kScanBlock];
    __shared__ int32_t total;
    int64_t i = int64_t(blockIdx.x) * kScanBlock + threadIdx.x;
    int32_t v = i < n ? in[i] : 0;
    int32_t ex = block_exclusive(v, lds, &total);
    if (i < n) out[i] = ex;
    __syncthreads();
    if (threadIdx.x == 0) block_sums[blockIdx.x] = total;
}

// Single workgroup: exclusive scan of the block sums, in chunks of 1024.
__global__ void __launch_bounds__(kScanBlock) scan_sums(int32_t *block_sums, int32_t n_blocks,
                                                        int32_t *grand_total) {
    __shared__ int32_t lds[kScanBlock];
    __shared__ int32_t total;
    int32_t carry = 0;
    for (int base = 0; base < n_blocks; base += kScanBlock) {
        int i = base + threadIdx.x;
        int32_t v = i < n_blocks ? block_sums[i] : 0;
        int32_t ex = block_exclusive(v, lds, &total);
        __syncthreads();
        if (i < n_blocks) block_sums[i] = ex + carry;
        carry += total;
        __syncthreads();
    }
    if (threadIdx.x == 0) *grand_total = carry;
}

__global__ void add_offsets(int32_t *out, int64_t n, const int32_t *block_sums,
                            const int32_t *grand_total) {
    int64_t i = int64_t(blockIdx.x) * kScanBlock + threadIdx.x;
    if (i < n) out[i] += block_sums[blockIdx.x];
    if (i == n) out[n] = *grand_total;
}
// Single workgroup, for short inputs: the input is staged in LDS with
// coalesced loads, thread t scans its own contiguous run of per elements
// there, the run totals are scanned across the block, and the runs are
// written back through LDS.  One launch instead of three.
constexpr int kOneBlockMax = kScanBlock * 16;
__global__ void __launch_bounds__(kScanBlock) scan_one_block(const int32_t *in, int32_t *out,
                                                             int n) {
    __shared__ int32_t lds[kScanBlock];
    __shared__ int32_t total;
    __shared__ int32_t buf[kOneBlockMax];
    for (int i = threadIdx.x; i < n; i += kScanBlock) buf[i] = in[i];
    __syncthreads();
    const int per = (n + kScanBlock - 1) / kScanBlock;
    const int lo = min(n, int(threadIdx.x) * per), hi = min(n, lo + per);
    int32_t run = 0;
    for (int i = lo; i < hi; ++i) run += buf[i];
    int32_t off = block_exclusive(run, lds, &total);
    for (int i = lo; i < hi; ++i) {
        const int32_t v = buf[i];
        buf[i] = off;
        off += v;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += kScanBlock) out[i] = buf[i];
    if (threadIdx.x == 0) out[n] = total;
}
}  // namespace

size_t scan_tmp_ints(int64_t n) { return size_t(ceil_div(n + 1, kScanBlock)) + 2; }

void exclusive_scan(const int32_t *in, int32_t *out, int64_t n, int32_t *tmp, hipStream_t s) {
    if (n <= kOneBlockMax) {
        hipLaunchKernelGGL(scan_one_block, dim3(1), dim3(kScanBlock), 0, s, in, out, int(n));
        RUNE_HIP_CHECK(hipGetLastError());
        return;
    }
    int nb = ceil_div(n + 1, kScanBlock);
    int32_t *sums = tmp;
    int32_t *grand = tmp + nb;
    hipLaunchKernelGGL(scan_blocks, dim3(nb), dim3(kScanBlock), 0, s, in, out, n, sums);
    hipLaunchKernelGGL(scan_sums, dim3(1), dim3(kScanBlock), 0, s, sums, nb, grand);
    hipLaunchKernelGGL(add_offsets, dim3(nb), dim3(kScanBlock), 0, s, out, n, sums, grand);
    RUNE_HIP_CHECK(hipGetLastError());
}

}  // namespace rune
