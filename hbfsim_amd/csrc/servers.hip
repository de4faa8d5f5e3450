// servers.hip -- k identical media servers with one read latency
// (src/prefetch/prefetch_model.cpp:22-50, MediaServers::issue) on the GPU.
//
// MediaServers keeps the k servers' free-at times in a min-heap, all 0 at
// the start; a read issued at `now` starts at max(now, earliest free) and
// completes L later.  Its caller issues reads at a clock that never runs
// backwards (simulate_prefetch, prefetch_model.cpp:124-186).  For such
// non-decreasing issue times the completions are non-decreasing too, and the
// server that frees first for read i is the one read i - k used, so
//   c_i = now_i + L                      (i < k)
//   c_i = max(now_i, c_{i-k}) + L        (i >= k),
// k interleaved Lindley chains.  Unrolled along a chain (q = i / k):
//   c_i = L (q_i + 1) + max_{j <= i, j = i mod k} (now_j - L q_j),
// a prefix maximum down each column of the n / k x k matrix of reads.
//
// Pipeline: transpose the reads to column order (computing w = now - L q),
// segmented prefix maximum over the columns (block summaries, a block-wide
// carry scan, then the blocks again), transpose back while adding L (q + 1).
// Out-of-order issue times are rejected (the heap and the chains differ
// then), found by a flag the transpose raises; so are times from 2^63 ns.
#include <hip/hip_runtime.h>

#include "engine.hpp"

#include <climits>
#include <cstdint>

namespace hbfamd {
namespace {

constexpr int kT = 64;         // transpose tile (kT x kT), 256 threads
constexpr int kScanB = 2048;   // elements per scan block (256 threads x 8)
constexpr int kCarryB = 1024;  // threads of the carry scan
constexpr std::int64_t kNegInf = INT64_MIN;

// rows x cols (row-major, n valid elements) -> w[c * rows + r] = now - L r
// (kNegInf past the end).  Also raises *bad when now decreases along the
// row-major order.
__global__ __launch_bounds__(256) void k_srv_in(const std::uint64_t* now, std::uint64_t n,
                                                std::uint64_t rows, std::uint64_t cols,
                                                std::uint64_t L, std::int64_t* w, int* bad)
{
    __shared__ std::int64_t tile[kT][kT + 1];
    const std::uint64_t r0 = static_cast<std::uint64_t>(blockIdx.x) * kT;
    const std::uint64_t c0 = static_cast<std::uint64_t>(blockIdx.y) * kT;
    const int tx = threadIdx.x % kT, ty = threadIdx.x / kT;  // 64 x 4
    for (int dy = ty; dy < kT; dy += 4) {
        const std::uint64_t r = r0 + dy, c = c0 + tx;
        std::int64_t v = kNegInf;
        if (r < rows && c < cols) {
            const std::uint64_t j = r * cols + c;
            if (j < n) {
                const std::uint64_t t = now[j];
                if ((j > 0 && now[j - 1] > t) || t > static_cast<std::uint64_t>(INT64_MAX)) {
                    atomicOr(bad, 1);
                }
                v = static_cast<std::int64_t>(t) - static_cast<std::int64_t>(L * r);
            }
        }
        tile[dy][tx] = v;
    }
    __syncthreads();
    for (int dx = ty; dx < kT; dx += 4) {
        const std::uint64_t c = c0 + dx, r = r0 + tx;
        if (c < cols && r < rows) {
            w[c * rows + r] = tile[tx][dx];
        }
    }
}

// Column order back to row order: out[r * cols + c] = L (r + 1) + m[c * rows + r].
__global__ __launch_bounds__(256) void k_srv_out(const std::int64_t* m, std::uint64_t n,
                                                 std::uint64_t rows, std::uint64_t cols,
                                                 std::uint64_t L, std::uint64_t* out)
{
    __shared__ std::int64_t tile[kT][kT + 1];
    const std::uint64_t r0 = static_cast<std::uint64_t>(blockIdx.x) * kT;
    const std::uint64_t c0 = static_cast<std::uint64_t>(blockIdx.y) * kT;
    const int tx = threadIdx.x % kT, ty = threadIdx.x / kT;
    for (int dx = ty; dx < kT; dx += 4) {
        const std::uint64_t c = c0 + dx, r = r0 + tx;
        tile[dx][tx] = (c < cols && r < rows) ? m[c * rows + r] : 0;
    }
    __syncthreads();
    for (int dy = ty; dy < kT; dy += 4) {
        const std::uint64_t r = r0 + dy, c = c0 + tx;
        if (r < rows && c < cols) {
            const std::uint64_t j = r * cols + c;
            if (j < n) {
                out[j] = L * (r + 1) + static_cast<std::uint64_t>(tile[tx][dy]);
            }
        }
    }
}

// Segmented maximum: segments are the columns (length `seg`).  A summary
// (head, m) is "the range holds a segment start" and the maximum after the
// last start (of the whole range if none); (h1, m1) then (h2, m2) is
// (h1 | h2, h2 ? m2 : max(m1, m2)).
struct SegMax {
    int head;
    std::int64_t m;
};

__device__ __forceinline__ SegMax seg_join(const SegMax& a, const SegMax& b)
{
    SegMax r;
    r.head = a.head | b.head;
    r.m = b.head ? b.m : (a.m > b.m ? a.m : b.m);
    return r;
}

// Inclusive block scan of SegMax over blockDim.x threads (Hillis-Steele).
template <int kThreads>
__device__ __forceinline__ SegMax block_scan(SegMax x, SegMax* sh)
{
    const int tid = threadIdx.x;
    sh[tid] = x;
    __syncthreads();
    for (int off = 1; off < kThreads; off <<= 1) {
        SegMax y{0, kNegInf};
        if (tid >= off) {
            y = sh[tid - off];
        }
        __syncthreads();
        x = seg_join(y, x);
        sh[tid] = x;
        __syncthreads();
    }
    return x;
}

// Pass 1 (kApply false): per block summary.  Pass 2 (kApply true): the
// running maximum from the block's carry-in, written back in place.
template <bool kApply>
__global__ __launch_bounds__(256) void k_srv_scan(std::int64_t* w, std::uint64_t total,
                                                  std::uint64_t seg, SegMax* bsum,
                                                  const SegMax* carry)
{
    __shared__ SegMax sh[256];
    const std::uint64_t b0 = static_cast<std::uint64_t>(blockIdx.x) * kScanB;
    const std::uint64_t e0 = b0 + static_cast<std::uint64_t>(threadIdx.x) * 8;
    std::int64_t v[8];
    SegMax own{0, kNegInf};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const std::uint64_t e = e0 + k;
        v[k] = e < total ? w[e] : kNegInf;
        const SegMax one{(e < total && e % seg == 0) ? 1 : 0, v[k]};
        own = seg_join(own, one);
    }
    const SegMax inc = block_scan<256>(own, sh);
    if (!kApply) {
        if (threadIdx.x == 255) {
            bsum[blockIdx.x] = inc;
        }
        return;
    }
    // exclusive prefix of this thread, from the block's carry-in
    SegMax run = carry[blockIdx.x];
    if (threadIdx.x > 0) {
        run = seg_join(run, sh[threadIdx.x - 1]);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const std::uint64_t e = e0 + k;
        const SegMax one{(e < total && e % seg == 0) ? 1 : 0, v[k]};
        run = seg_join(run, one);
        if (e < total) {
            w[e] = run.m;
        }
    }
}

// Exclusive scan of the block summaries (one block, kCarryB per pass).
__global__ __launch_bounds__(kCarryB) void k_srv_carry(const SegMax* bsum, std::uint64_t nb,
                                                       SegMax* carry)
{
    __shared__ SegMax sh[kCarryB];
    __shared__ SegMax next;
    SegMax run{0, kNegInf};
    for (std::uint64_t b0 = 0; b0 < nb; b0 += kCarryB) {
        const std::uint64_t b = b0 + threadIdx.x;
        const SegMax own = b < nb ? bsum[b] : SegMax{0, kNegInf};
        const SegMax inc = block_scan<kCarryB>(own, sh);
        SegMax before = run;
        if (threadIdx.x > 0) {
            before = seg_join(run, sh[threadIdx.x - 1]);
        }
        if (b < nb) {
            carry[b] = before;
        }
        if (threadIdx.x == kCarryB - 1) {
            next = seg_join(run, inc);
        }
        __syncthreads();
        run = next;
        __syncthreads();
    }
}

}  // namespace

int media_servers(const std::uint64_t* d_now, std::size_t n, std::uint32_t servers,
                  std::uint64_t latency_ns, std::uint64_t* d_completion, void* stream_ptr)
{
    if (n == 0) {
        return HBFSIM_OK;
    }
    if (d_now == nullptr || d_completion == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const std::uint64_t k = servers == 0 ? 1 : servers;
    const std::uint64_t cols = k < n ? k : n;
    const std::uint64_t rows = (n + cols - 1) / cols;
    const std::uint64_t total = rows * cols;
    const std::uint64_t nb = (total + kScanB - 1) / kScanB;
    if (rows > 0x7fffffffull || (cols + kT - 1) / kT > 65535 ||
        latency_ns > static_cast<std::uint64_t>(INT64_MAX) / (rows + 1)) {
        return HBFSIM_UNSUPPORTED;
    }
    std::int64_t* w = nullptr;
    SegMax* bsum = nullptr;
    SegMax* carry = nullptr;
    int* bad = nullptr;
    int h_bad = 0;
    hipError_t err = hipMalloc(reinterpret_cast<void**>(&w), total * sizeof(std::int64_t));
    if (err == hipSuccess) err = hipMalloc(reinterpret_cast<void**>(&bsum), nb * sizeof(SegMax));
    if (err == hipSuccess) err = hipMalloc(reinterpret_cast<void**>(&carry), nb * sizeof(SegMax));
    if (err == hipSuccess) err = hipMalloc(reinterpret_cast<void**>(&bad), sizeof(int));
    if (err == hipSuccess) err = hipMemsetAsync(bad, 0, sizeof(int), stream);
    if (err == hipSuccess) {
        const dim3 tg(static_cast<unsigned>((rows + kT - 1) / kT),
                      static_cast<unsigned>((cols + kT - 1) / kT));
        hipLaunchKernelGGL(k_srv_in, tg, dim3(256), 0, stream, d_now, n, rows, cols, latency_ns,
                           w, bad);
        hipLaunchKernelGGL((k_srv_scan<false>), dim3(static_cast<unsigned>(nb)), dim3(256), 0,
                           stream, w, total, rows, bsum, static_cast<const SegMax*>(nullptr));
        hipLaunchKernelGGL(k_srv_carry, dim3(1), dim3(kCarryB), 0, stream, bsum, nb, carry);
        hipLaunchKernelGGL((k_srv_scan<true>), dim3(static_cast<unsigned>(nb)), dim3(256), 0,
                           stream, w, total, rows, static_cast<SegMax*>(nullptr), carry);
        hipLaunchKernelGGL(k_srv_out, tg, dim3(256), 0, stream, w, n, rows, cols, latency_ns,
                           d_completion);
        err = hipGetLastError();
    }
    if (err == hipSuccess) err = hipMemcpyAsync(&h_bad, bad, sizeof(int), hipMemcpyDeviceToHost,
                                                stream);
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    (void)hipFree(w);
    (void)hipFree(bsum);
    (void)hipFree(carry);
    (void)hipFree(bad);
    if (err != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    return h_bad != 0 ? HBFSIM_INVALID_ARGUMENT : HBFSIM_OK;
}

}  // namespace hbfamd
