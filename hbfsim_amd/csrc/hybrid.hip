// hybrid.hip -- the hybrid model's request sampler and calibrator
// (src/hybrid/calibrator.cpp:67-138) on the GPU.
//
// HybridSampler::reference(sequence, access) (calibrator.cpp:83-96) sends a
// request to the detailed model when its sequence is a warm-up one, when its
// access class was never seen before, or when a SplitMix64 hash of
// (sequence, seed, class) falls at or below the rate's threshold.  Over a
// batch the "never seen" requests are the first occurrence of each class in
// the batch whose class is also absent from the classes earlier batches saw.
//
// Calibrator (calibrator.cpp:98-136) keeps every latency per class and
// reports count, mean, p50/p95/p99 and the mean and deviation of the logs.
//
// Both sort the batch by class with stable LSD radix passes over 64-bit
// keys (hi = operation:bytes, lo = queue:locality, and for the calibrator the
// latency below them), so a class occupies one contiguous segment, its
// requests in their original order (sampler) or its latencies ascending
// (calibrator).  Segment heads are then the first occurrences and the
// calibrator's per-class rows come out in the class order of the reference's
// std::map.
#include <hip/hip_runtime.h>

#include <cstring>  // rocPRIM's host code uses memset
#include <rocprim/device/device_radix_sort.hpp>

#include "engine.hpp"

#include <cmath>
#include <cstdint>
#include <limits>

namespace hbfamd {
namespace {

constexpr int kThreads = 256;
constexpr int kRowThreads = 256;

__device__ __forceinline__ std::uint64_t class_hi(const hbfsim_amd_access_class& c)
{
    return (static_cast<std::uint64_t>(c.operation) << 32) | c.bytes;
}

__device__ __forceinline__ std::uint64_t class_lo(const hbfsim_amd_access_class& c)
{
    return (static_cast<std::uint64_t>(c.queue_bucket) << 32) | c.locality_bucket;
}

// SplitMix64 finaliser (calibrator.cpp:12-18).
__device__ __forceinline__ std::uint64_t mix(std::uint64_t v)
{
    v += 0x9e3779b97f4a7c15ull;
    v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ull;
    v = (v ^ (v >> 27)) * 0x94d049bb133111ebull;
    return v ^ (v >> 31);
}

unsigned blocks_for(std::size_t n)
{
    return static_cast<unsigned>((n + kThreads - 1) / kThreads);
}

// key[i] = the class's low key (or latency[i] when given), idx[i] = i.
__global__ __launch_bounds__(kThreads) void k_first_keys(const hbfsim_amd_access_class* access,
                                                         const std::uint64_t* latency,
                                                         std::size_t n, std::uint64_t* key,
                                                         std::uint32_t* idx, int* bad)
{
    const std::size_t i = static_cast<std::size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= n) {
        return;
    }
    if (latency != nullptr) {
        const std::uint64_t v = latency[i];
        if (v == 0) {
            atomicOr(bad, 1);
        }
        key[i] = v;
    } else {
        key[i] = class_lo(access[i]);
    }
    idx[i] = static_cast<std::uint32_t>(i);
}

// key[j] = hi or lo class key of request idx[j].
template <bool kHi>
__global__ __launch_bounds__(kThreads) void k_gather_keys(const hbfsim_amd_access_class* access,
                                                          const std::uint32_t* idx,
                                                          std::size_t n, std::uint64_t* key)
{
    const std::size_t j = static_cast<std::size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (j < n) {
        const hbfsim_amd_access_class c = access[idx[j]];
        key[j] = kHi ? class_hi(c) : class_lo(c);
    }
}

__device__ __forceinline__ bool same_class(const hbfsim_amd_access_class& a,
                                           const hbfsim_amd_access_class& b)
{
    return a.operation == b.operation && a.bytes == b.bytes &&
           a.queue_bucket == b.queue_bucket && a.locality_bucket == b.locality_bucket;
}

// flags[i] = warm-up or hash decision (calibrator.cpp:86-95); counts are
// taken after the first-occurrence pass.
__global__ __launch_bounds__(kThreads) void k_sampler_decide(
    const hbfsim_amd_access_class* access, const std::uint64_t* sequence,
    std::uint64_t first_sequence, std::size_t n, std::uint32_t warmup,
    std::uint64_t threshold, std::uint64_t seed, std::uint8_t* flags)
{
    const std::size_t i = static_cast<std::size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= n) {
        return;
    }
    const hbfsim_amd_access_class c = access[i];
    const std::uint64_t s = sequence != nullptr ? sequence[i] : first_sequence + i;
    std::uint64_t v = s ^ seed;
    v ^= static_cast<std::uint64_t>(c.bytes) << 17;
    v ^= static_cast<std::uint64_t>(c.queue_bucket) << 33;
    v ^= static_cast<std::uint64_t>(c.locality_bucket) << 49;
    v ^= static_cast<std::uint64_t>(c.operation) << 61;
    flags[i] = (s < warmup || mix(v) <= threshold) ? 1 : 0;
}

// Lower bound of (hi, lo) in the seen set, sorted by (hi, lo).
__device__ __forceinline__ bool seen_contains(const std::uint64_t* seen_hi,
                                              const std::uint64_t* seen_lo, std::size_t count,
                                              std::uint64_t hi, std::uint64_t lo)
{
    std::size_t lo_i = 0, hi_i = count;
    while (lo_i < hi_i) {
        const std::size_t mid = lo_i + (hi_i - lo_i) / 2;
        const bool less = seen_hi[mid] < hi || (seen_hi[mid] == hi && seen_lo[mid] < lo);
        if (less) {
            lo_i = mid + 1;
        } else {
            hi_i = mid;
        }
    }
    return lo_i < count && seen_hi[lo_i] == hi && seen_lo[lo_i] == lo;
}

// Segment heads of the class-sorted batch: the first request of a class
// not in the seen set is a reference request, and its class joins the set.
__global__ __launch_bounds__(kThreads) void k_sampler_heads(
    const hbfsim_amd_access_class* access, const std::uint32_t* idx, std::size_t n,
    const std::uint64_t* seen_hi, const std::uint64_t* seen_lo, std::size_t seen,
    std::uint8_t* flags, std::uint64_t* new_hi, std::uint64_t* new_lo,
    unsigned long long* new_count)
{
    const std::size_t j = static_cast<std::size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (j >= n) {
        return;
    }
    const std::uint32_t i = idx[j];
    const hbfsim_amd_access_class c = access[i];
    if (j > 0 && same_class(access[idx[j - 1]], c)) {
        return;
    }
    const std::uint64_t hi = class_hi(c), lo = class_lo(c);
    if (!seen_contains(seen_hi, seen_lo, seen, hi, lo)) {
        flags[i] = 1;
        const unsigned long long k = atomicAdd(new_count, 1ull);
        new_hi[k] = hi;
        new_lo[k] = lo;
    }
}

// Sum of flags into *count (one atomic per block).
__global__ __launch_bounds__(kThreads) void k_count_flags(const std::uint8_t* flags,
                                                          std::size_t n,
                                                          unsigned long long* count)
{
    __shared__ unsigned partial[kThreads / 64];
    const std::size_t i = static_cast<std::size_t>(blockIdx.x) * kThreads + threadIdx.x;
    unsigned v = (i < n && flags[i] != 0) ? 1u : 0u;
    for (int off = 32; off > 0; off >>= 1) {
        v += __shfl_down(v, off);
    }
    if ((threadIdx.x & 63) == 0) {
        partial[threadIdx.x / 64] = v;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned s = 0;
        for (int w = 0; w < kThreads / 64; ++w) {
            s += partial[w];
        }
        if (s != 0) {
            atomicAdd(count, static_cast<unsigned long long>(s));
        }
    }
}

// Segment starts of the class-sorted batch, in no particular order.
__global__ __launch_bounds__(kThreads) void k_segment_starts(
    const hbfsim_amd_access_class* access, const std::uint32_t* idx, std::size_t n,
    std::uint32_t* starts, unsigned long long* count)
{
    const std::size_t j = static_cast<std::size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (j >= n) {
        return;
    }
    if (j == 0 || !same_class(access[idx[j - 1]], access[idx[j]])) {
        const unsigned long long k = atomicAdd(count, 1ull);
        starts[k] = static_cast<std::uint32_t>(j);
    }
}

// 128-bit sum as two 64-bit words.
struct U128 {
    std::uint64_t lo, hi;
};

__device__ __forceinline__ U128 add128(U128 a, U128 b)
{
    U128 r;
    r.lo = a.lo + b.lo;
    r.hi = a.hi + b.hi + (r.lo < a.lo ? 1ull : 0ull);
    return r;
}

// floor(s / d) for d < 2^32 and a quotient below 2^64, in 32-bit digits.
__device__ __forceinline__ std::uint64_t div128(U128 s, std::uint64_t d)
{
    const std::uint64_t digit[4] = {s.hi >> 32, s.hi & 0xffffffffull, s.lo >> 32,
                                    s.lo & 0xffffffffull};
    std::uint64_t r = 0, q = 0;
    for (int k = 0; k < 4; ++k) {
        const std::uint64_t cur = (r << 32) | digit[k];
        q = (q << 32) | (cur / d);
        r = cur % d;
    }
    return q;
}

template <typename T, typename Op>
__device__ __forceinline__ T block_reduce(T v, T* sh, Op op)
{
    sh[threadIdx.x] = v;
    __syncthreads();
    for (int off = kRowThreads / 2; off > 0; off >>= 1) {
        if (static_cast<int>(threadIdx.x) < off) {
            sh[threadIdx.x] = op(sh[threadIdx.x], sh[threadIdx.x + off]);
        }
        __syncthreads();
    }
    const T r = sh[0];
    __syncthreads();
    return r;
}

// calibrator.cpp:20-30: the sample of rank ceil(size * num / den), 1-based,
// clamped to the segment.
__device__ __forceinline__ std::uint64_t rank_index(std::uint64_t size, std::uint32_t num,
                                                    std::uint32_t den)
{
    const std::uint64_t rank = (size * num + den - 1) / den;
    const std::uint64_t index = rank == 0 ? 0 : rank - 1;
    return index < size - 1 ? index : size - 1;
}

// One block per class segment [starts[b], starts[b + 1]) of the sorted
// latencies: the estimate of calibrator.cpp:107-136.  The logs are summed
// in double by a fixed tree, so the result depends only on the samples.
__global__ __launch_bounds__(kRowThreads) void k_calib_rows(
    const hbfsim_amd_access_class* access, const std::uint32_t* idx, const std::uint64_t* lat,
    const std::uint32_t* starts, std::size_t classes, std::size_t n,
    hbfsim_amd_calibration* rows)
{
    __shared__ U128 sh_sum[kRowThreads];
    __shared__ double sh_d[kRowThreads];
    const std::size_t b = blockIdx.x;
    const std::size_t s = starts[b];
    const std::size_t e = b + 1 < classes ? starts[b + 1] : n;
    const std::uint64_t size = e - s;
    U128 sum{0, 0};
    double log_sum = 0.0;
    for (std::size_t k = s + threadIdx.x; k < e; k += kRowThreads) {
        const std::uint64_t v = lat[k];
        sum = add128(sum, U128{v, 0});
        log_sum += log(static_cast<double>(v));
    }
    sum = block_reduce(sum, sh_sum, [](U128 x, U128 y) { return add128(x, y); });
    log_sum = block_reduce(log_sum, sh_d, [](double x, double y) { return x + y; });
    const double log_mean = log_sum / static_cast<double>(size);
    double squared = 0.0;
    for (std::size_t k = s + threadIdx.x; k < e; k += kRowThreads) {
        const double delta = log(static_cast<double>(lat[k])) - log_mean;
        squared += delta * delta;
    }
    squared = block_reduce(squared, sh_d, [](double x, double y) { return x + y; });
    if (threadIdx.x == 0) {
        hbfsim_amd_calibration r;
        r.access = access[idx[s]];
        r.count = size;
        r.mean_ns = div128(sum, size);
        r.p50_ns = lat[s + rank_index(size, 50, 100)];
        r.p95_ns = lat[s + rank_index(size, 95, 100)];
        r.p99_ns = lat[s + rank_index(size, 99, 100)];
        r.log_mean = log_mean;
        r.log_sigma = sqrt(squared / static_cast<double>(size));
        rows[b] = r;
    }
}

// Device buffers of one call, freed on scope exit.
struct Buffers {
    void* p[10]{};
    int used = 0;
    hipError_t err = hipSuccess;
    template <typename T>
    T* get(std::size_t count)
    {
        void* q = nullptr;
        if (err == hipSuccess) {
            err = hipMalloc(&q, count == 0 ? 1 : count * sizeof(T));
        }
        if (err == hipSuccess) {
            p[used++] = q;
        }
        return static_cast<T*>(q);
    }
    ~Buffers()
    {
        for (int k = 0; k < used; ++k) {
            (void)hipFree(p[k]);
        }
    }
};

__global__ __launch_bounds__(kThreads) void k_iota(std::uint32_t* idx, std::size_t n)
{
    const std::size_t i = static_cast<std::size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i < n) {
        idx[i] = static_cast<std::uint32_t>(i);
    }
}

__global__ __launch_bounds__(kThreads) void k_gather_u64(const std::uint64_t* src,
                                                         const std::uint32_t* idx,
                                                         std::size_t n, std::uint64_t* out)
{
    const std::size_t j = static_cast<std::size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (j < n) {
        out[j] = src[idx[j]];
    }
}

// Stable sort of request indices by class, and by latency inside a class
// when `latency` is given: LSD passes (latency,) low class key, high class
// key, each a stable radix sort carrying the permutation.  key_a/key_b and
// idx_a/idx_b are n-entry ping-pong buffers; *perm receives whichever of
// idx_a/idx_b holds the final permutation.
hipError_t sort_by_class(const hbfsim_amd_access_class* access, const std::uint64_t* latency,
                         std::size_t n, std::uint64_t* key_a, std::uint64_t* key_b,
                         std::uint32_t* idx_a, std::uint32_t* idx_b, void* temp,
                         std::size_t temp_bytes, int* bad, std::uint32_t** perm,
                         hipStream_t stream)
{
    const unsigned grid = blocks_for(n);
    std::size_t tb = temp_bytes;
    hipLaunchKernelGGL(k_first_keys, dim3(grid), dim3(kThreads), 0, stream, access, latency, n,
                       key_a, idx_a, bad);
    hipError_t err = hipGetLastError();
    if (err == hipSuccess) {
        err = rocprim::radix_sort_pairs(temp, tb, key_a, key_b, idx_a, idx_b, n, 0, 64, stream);
    }
    std::uint32_t* p = idx_b;  // current permutation
    std::uint32_t* q = idx_a;  // the other buffer
    if (latency != nullptr && err == hipSuccess) {
        hipLaunchKernelGGL((k_gather_keys<false>), dim3(grid), dim3(kThreads), 0, stream, access,
                           p, n, key_a);
        err = rocprim::radix_sort_pairs(temp, tb, key_a, key_b, p, q, n, 0, 64, stream);
        std::swap(p, q);
    }
    if (err == hipSuccess) {
        hipLaunchKernelGGL((k_gather_keys<true>), dim3(grid), dim3(kThreads), 0, stream, access,
                           p, n, key_a);
        err = rocprim::radix_sort_pairs(temp, tb, key_a, key_b, p, q, n, 0, 64, stream);
        std::swap(p, q);
    }
    if (err == hipSuccess) {
        err = hipGetLastError();
    }
    *perm = p;
    return err;
}

hipError_t sort_temp_bytes(std::size_t n, std::size_t* bytes)
{
    return rocprim::radix_sort_pairs(nullptr, *bytes, static_cast<std::uint64_t*>(nullptr),
                                     static_cast<std::uint64_t*>(nullptr),
                                     static_cast<std::uint32_t*>(nullptr),
                                     static_cast<std::uint32_t*>(nullptr), n, 0, 64);
}

// Latencies gathered into class order for the calibrator: lat_sorted[j] =
// latency of request idx[j].  (The latency sort ran first, so within a
// class they ascend.)
__global__ __launch_bounds__(kThreads) void k_gather_latency(const std::uint64_t* latency,
                                                             const std::uint32_t* idx,
                                                             std::size_t n, std::uint64_t* out)
{
    const std::size_t j = static_cast<std::size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (j < n) {
        out[j] = latency[idx[j]];
    }
}

}  // namespace

struct sampler_state {
    std::uint32_t warmup;
    std::uint64_t threshold;
    std::uint64_t seed;
    std::uint64_t* seen_hi = nullptr;  // seen classes, sorted by (hi, lo)
    std::uint64_t* seen_lo = nullptr;
    std::size_t seen = 0;
    std::size_t seen_cap = 0;
};

int sampler_create(std::uint32_t warmup, double sample_rate, std::uint64_t seed,
                   sampler_state** out)
{
    if (out == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    *out = nullptr;
    // calibrator.cpp:67-81
    if (!std::isfinite(sample_rate) || sample_rate < 0.0 || sample_rate > 1.0) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    auto* s = new (std::nothrow) sampler_state;
    if (s == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    s->warmup = warmup;
    s->seed = seed;
    s->threshold = sample_rate >= 1.0
                       ? std::numeric_limits<std::uint64_t>::max()
                       : static_cast<std::uint64_t>(
                             sample_rate * static_cast<long double>(
                                               std::numeric_limits<std::uint64_t>::max()));
    *out = s;
    return HBFSIM_OK;
}

void sampler_destroy(sampler_state* s)
{
    if (s != nullptr) {
        (void)hipFree(s->seen_hi);
        (void)hipFree(s->seen_lo);
        delete s;
    }
}

int sampler_reference(sampler_state* s, const hbfsim_amd_access_class* d_access,
                      const std::uint64_t* d_sequence, std::uint64_t first_sequence,
                      std::size_t n, std::uint8_t* d_flags, std::uint64_t* references,
                      void* stream_ptr)
{
    if (s == nullptr || (n != 0 && (d_access == nullptr || d_flags == nullptr))) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    if (references != nullptr) {
        *references = 0;
    }
    if (n == 0) {
        return HBFSIM_OK;
    }
    if (n > 0xffffffffull) {
        return HBFSIM_UNSUPPORTED;
    }
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    std::size_t temp_bytes = 0;
    hipError_t err = sort_temp_bytes(n, &temp_bytes);
    Buffers buf;
    auto* key_a = buf.get<std::uint64_t>(n);
    auto* key_b = buf.get<std::uint64_t>(n);
    auto* idx_a = buf.get<std::uint32_t>(n);
    auto* idx_b = buf.get<std::uint32_t>(n);
    void* temp = buf.get<unsigned char>(temp_bytes);
    auto* counters = buf.get<unsigned long long>(2);  // new classes, references
    int* bad = buf.get<int>(1);
    if (err == hipSuccess) err = buf.err;
    if (err == hipSuccess) err = hipMemsetAsync(counters, 0, 2 * sizeof(unsigned long long),
                                                stream);
    std::uint32_t* perm = nullptr;
    if (err == hipSuccess) {
        err = sort_by_class(d_access, nullptr, n, key_a, key_b, idx_a, idx_b, temp, temp_bytes,
                            bad, &perm, stream);
    }
    // perm: requests in class order; key_a/key_b are free again and take
    // the new classes.
    const unsigned grid = blocks_for(n);
    if (err == hipSuccess) {
        hipLaunchKernelGGL(k_sampler_decide, dim3(grid), dim3(kThreads), 0, stream, d_access,
                           d_sequence, first_sequence, n, s->warmup, s->threshold, s->seed,
                           d_flags);
        hipLaunchKernelGGL(k_sampler_heads, dim3(grid), dim3(kThreads), 0, stream, d_access,
                           perm, n, s->seen_hi, s->seen_lo, s->seen, d_flags, key_a, key_b,
                           counters);
        hipLaunchKernelGGL(k_count_flags, dim3(grid), dim3(kThreads), 0, stream, d_flags, n,
                           counters + 1);
        err = hipGetLastError();
    }
    unsigned long long host[2] = {0, 0};
    if (err == hipSuccess) err = hipMemcpyAsync(host, counters, sizeof(host),
                                                hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    if (err == hipSuccess && host[0] != 0) {
        // seen := sort(seen + new) by (hi, lo)
        const std::size_t total = s->seen + host[0];
        std::size_t tb2 = 0;
        err = sort_temp_bytes(total, &tb2);
        Buffers b2;
        auto* hi_a = b2.get<std::uint64_t>(total);
        auto* lo_a = b2.get<std::uint64_t>(total);
        auto* hi_b = b2.get<std::uint64_t>(total);
        auto* lo_b = b2.get<std::uint64_t>(total);
        auto* ia = b2.get<std::uint32_t>(total);
        auto* ib = b2.get<std::uint32_t>(total);
        void* t2 = b2.get<unsigned char>(tb2);
        if (err == hipSuccess) err = b2.err;
        std::uint64_t* nh = nullptr;
        std::uint64_t* nl = nullptr;
        if (err == hipSuccess) err = hipMalloc(reinterpret_cast<void**>(&nh), total * 8);
        if (err == hipSuccess) err = hipMalloc(reinterpret_cast<void**>(&nl), total * 8);
        if (err == hipSuccess && s->seen != 0) {
            err = hipMemcpyAsync(hi_a, s->seen_hi, s->seen * 8, hipMemcpyDeviceToDevice, stream);
            if (err == hipSuccess) err = hipMemcpyAsync(lo_a, s->seen_lo, s->seen * 8,
                                                        hipMemcpyDeviceToDevice, stream);
        }
        if (err == hipSuccess) err = hipMemcpyAsync(hi_a + s->seen, key_a, host[0] * 8,
                                                    hipMemcpyDeviceToDevice, stream);
        if (err == hipSuccess) err = hipMemcpyAsync(lo_a + s->seen, key_b, host[0] * 8,
                                                    hipMemcpyDeviceToDevice, stream);
        // By lo, then stably by hi; the payload is the position in hi_a/lo_a.
        std::size_t tb = tb2;
        if (err == hipSuccess) {
            hipLaunchKernelGGL(k_iota, dim3(blocks_for(total)), dim3(kThreads), 0, stream, ia,
                               total);
            err = rocprim::radix_sort_pairs(t2, tb, lo_a, lo_b, ia, ib, total, 0, 64, stream);
        }
        if (err == hipSuccess) {
            hipLaunchKernelGGL(k_gather_u64, dim3(blocks_for(total)), dim3(kThreads), 0, stream,
                               hi_a, ib, total, hi_b);
            err = rocprim::radix_sort_pairs(t2, tb, hi_b, nh, ib, ia, total, 0, 64, stream);
        }
        if (err == hipSuccess) {
            hipLaunchKernelGGL(k_gather_u64, dim3(blocks_for(total)), dim3(kThreads), 0, stream,
                               lo_a, ia, total, nl);
            err = hipGetLastError();
        }
        if (err == hipSuccess) err = hipStreamSynchronize(stream);
        if (err == hipSuccess) {
            (void)hipFree(s->seen_hi);
            (void)hipFree(s->seen_lo);
            s->seen_hi = nh;
            s->seen_lo = nl;
            s->seen = total;
        } else {
            (void)hipFree(nh);
            (void)hipFree(nl);
        }
    }
    if (err != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    if (references != nullptr) {
        *references = host[1];
    }
    return HBFSIM_OK;
}

int calibrate(const hbfsim_amd_access_class* d_access, const std::uint64_t* d_latency,
              std::size_t n, hbfsim_amd_calibration* d_rows, std::size_t max_rows,
              std::size_t* rows_out, void* stream_ptr)
{
    if (rows_out == nullptr || (n != 0 && (d_access == nullptr || d_latency == nullptr))) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    *rows_out = 0;
    if (n == 0) {
        return HBFSIM_OK;
    }
    if (n > 0xffffffffull) {
        return HBFSIM_UNSUPPORTED;
    }
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    std::size_t temp_bytes = 0;
    hipError_t err = sort_temp_bytes(n, &temp_bytes);
    Buffers buf;
    auto* key_a = buf.get<std::uint64_t>(n);
    auto* key_b = buf.get<std::uint64_t>(n);
    auto* idx_a = buf.get<std::uint32_t>(n);
    auto* idx_b = buf.get<std::uint32_t>(n);
    void* temp = buf.get<unsigned char>(temp_bytes);
    auto* counters = buf.get<unsigned long long>(1);
    int* bad = buf.get<int>(1);
    if (err == hipSuccess) err = buf.err;
    if (err == hipSuccess) err = hipMemsetAsync(counters, 0, sizeof(unsigned long long), stream);
    if (err == hipSuccess) err = hipMemsetAsync(bad, 0, sizeof(int), stream);
    std::uint32_t* perm = nullptr;
    if (err == hipSuccess) {
        err = sort_by_class(d_access, d_latency, n, key_a, key_b, idx_a, idx_b, temp, temp_bytes,
                            bad, &perm, stream);
    }
    // perm: class order, latencies ascending inside a class.  key_a takes
    // the sorted latencies, the other index buffer the segment starts
    // (unordered), key_b (as 2n 32-bit words) the ordered starts.
    std::uint32_t* starts_raw = perm == idx_a ? idx_b : idx_a;
    auto* starts = reinterpret_cast<std::uint32_t*>(key_b);
    const unsigned grid = blocks_for(n);
    if (err == hipSuccess) {
        hipLaunchKernelGGL(k_gather_latency, dim3(grid), dim3(kThreads), 0, stream, d_latency,
                           perm, n, key_a);
        hipLaunchKernelGGL(k_segment_starts, dim3(grid), dim3(kThreads), 0, stream, d_access,
                           perm, n, starts_raw, counters);
        err = hipGetLastError();
    }
    unsigned long long classes = 0;
    int h_bad = 0;
    if (err == hipSuccess) err = hipMemcpyAsync(&classes, counters, sizeof(classes),
                                                hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess) err = hipMemcpyAsync(&h_bad, bad, sizeof(int),
                                                hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    if (err != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    if (h_bad != 0) {
        return HBFSIM_INVALID_ARGUMENT;  // Calibrator::observe: latency_ns must be positive
    }
    *rows_out = classes;
    if (classes > max_rows || d_rows == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    // starts in ascending order
    std::size_t tb = 0;
    err = rocprim::radix_sort_keys(nullptr, tb, starts_raw, starts,
                                   static_cast<std::size_t>(classes), 0, 32, stream);
    Buffers b2;
    void* t2 = b2.get<unsigned char>(tb);
    if (err == hipSuccess) err = b2.err;
    if (err == hipSuccess) {
        err = rocprim::radix_sort_keys(t2, tb, starts_raw, starts,
                                       static_cast<std::size_t>(classes), 0, 32, stream);
    }
    if (err == hipSuccess) {
        hipLaunchKernelGGL(k_calib_rows, dim3(static_cast<unsigned>(classes)), dim3(kRowThreads),
                           0, stream, d_access, perm, key_a, starts,
                           static_cast<std::size_t>(classes), n, d_rows);
        err = hipGetLastError();
    }
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    return err == hipSuccess ? HBFSIM_OK : HBFSIM_CUDA_ERROR;
}

}  // namespace hbfamd
