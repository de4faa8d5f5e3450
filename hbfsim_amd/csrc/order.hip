// order.hip -- issue-time order of a record stream (gfx950).
//
// The engine serves every resource in (issue time, stream position) order,
// the order in which the reference's MQSim adapter serves staged arrivals:
// sorted by (arrival, sequence) (src/mqsim_adapter/mqsim_online.cpp:
// 269-289).  Streams that are already issue-ordered (every workload
// generator's) are timed as they lie; the main pipeline notices any record
// whose issue time goes back while it summarises its tiles, and the engine
// then times the stream once more from a copy sorted here: the issue times
// are radix-sorted with the record positions as payload (rocPRIM's LSD radix
// sort is stable, so equal issue times keep stream order), the records are
// gathered into that order, timed, and their completion times and status
// bytes are scattered back to their stream positions.
#include <hip/hip_runtime.h>

#include <cstring>  // rocPRIM's host code uses memset
#include <rocprim/device/device_radix_sort.hpp>

#include "engine.hpp"

#include <cstdint>

namespace hbfamd {
namespace {

constexpr int kThreads = 256;
constexpr unsigned kMaxBlocks = 65536;

// Issue time of record i: 32-byte records hold it in word 2; packed records
// in bits 0-55 of their second word.
template <bool kPacked>
__device__ __forceinline__ std::uint64_t issue_of(const void* rec, std::size_t i)
{
    if (kPacked) {
        const std::uint64_t w = static_cast<const hbf_record16*>(rec)[i].issue_op;
        return w & ((1ull << 56) - 1);
    }
    return static_cast<const hbf_record32*>(rec)[i].issue_ps;
}

unsigned blocks_for(std::size_t n)
{
    const std::size_t b = (n + kThreads - 1) / kThreads;
    return static_cast<unsigned>(b < kMaxBlocks ? (b == 0 ? 1 : b) : kMaxBlocks);
}

// *flag = 1 when some record's issue time is below its predecessor's.
template <bool kPacked>
__global__ __launch_bounds__(kThreads) void k_order_check(const void* rec, std::size_t n,
                                                          std::uint32_t* flag)
{
    const std::size_t stride = static_cast<std::size_t>(gridDim.x) * kThreads;
    bool bad = false;
    for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * kThreads + threadIdx.x + 1; i < n;
         i += stride) {
        bad = bad || issue_of<kPacked>(rec, i) < issue_of<kPacked>(rec, i - 1);
    }
    if (bad) {
        *flag = 1u;
    }
}

template <bool kPacked>
__global__ __launch_bounds__(kThreads) void k_issue_keys(const void* rec, std::size_t n,
                                                         std::uint64_t* keys, std::uint32_t* pos)
{
    const std::size_t stride = static_cast<std::size_t>(gridDim.x) * kThreads;
    for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += stride) {
        keys[i] = issue_of<kPacked>(rec, i);
        pos[i] = static_cast<std::uint32_t>(i);
    }
}

// out[j] = rec[pos[j]] (T: hbf_record32 or hbf_record16).
template <typename T>
__global__ __launch_bounds__(kThreads) void k_gather_records(const T* rec,
                                                             const std::uint32_t* pos,
                                                             std::size_t n, T* out)
{
    const std::size_t stride = static_cast<std::size_t>(gridDim.x) * kThreads;
    for (std::size_t j = static_cast<std::size_t>(blockIdx.x) * kThreads + threadIdx.x; j < n;
         j += stride) {
        out[j] = rec[pos[j]];
    }
}

// comp[pos[j]] = scomp[j], status[pos[j]] = sstatus[j] (status optional).
__global__ __launch_bounds__(kThreads) void k_scatter(const std::uint32_t* pos, std::size_t n,
                                                      const std::uint64_t* scomp,
                                                      const std::uint8_t* sstatus,
                                                      std::uint64_t* comp, std::uint8_t* status)
{
    const std::size_t stride = static_cast<std::size_t>(gridDim.x) * kThreads;
    for (std::size_t j = static_cast<std::size_t>(blockIdx.x) * kThreads + threadIdx.x; j < n;
         j += stride) {
        const std::uint32_t i = pos[j];
        comp[i] = scomp[j];
        if (status != nullptr) {
            status[i] = sstatus[j];
        }
    }
}

template <typename T>
hipError_t dalloc(T*& p, std::size_t count)
{
    return hipMalloc(reinterpret_cast<void**>(&p), sizeof(T) * (count == 0 ? 1 : count));
}

template <typename T>
void dfree(T*& p)
{
    if (p != nullptr) {
        (void)hipFree(p);
        p = nullptr;
    }
}

}  // namespace

int order_check(const void* d_rec, bool packed, std::size_t n, std::uint32_t* d_flag,
                void* stream_ptr)
{
    if (n < 2) {
        return HBFSIM_OK;
    }
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    if (packed) {
        hipLaunchKernelGGL(k_order_check<true>, dim3(blocks_for(n)), dim3(kThreads), 0, stream,
                           d_rec, n, d_flag);
    } else {
        hipLaunchKernelGGL(k_order_check<false>, dim3(blocks_for(n)), dim3(kThreads), 0, stream,
                           d_rec, n, d_flag);
    }
    return hipGetLastError() == hipSuccess ? HBFSIM_OK : HBFSIM_CUDA_ERROR;
}

int run_in_issue_order(const void* d_rec, bool packed, std::size_t n, std::uint64_t* d_comp,
                       std::uint8_t* d_status, void* stream_ptr, const sorted_runner& run)
{
    if (n >= (1ull << 32)) {
        return HBFSIM_UNSUPPORTED;  // positions travel as 32-bit payload
    }
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const std::size_t rec_bytes = packed ? sizeof(hbf_record16) : sizeof(hbf_record32);
    std::uint64_t* keys_a = nullptr;
    std::uint64_t* keys_b = nullptr;
    std::uint32_t* pos_a = nullptr;
    std::uint32_t* pos_b = nullptr;
    void* temp = nullptr;
    unsigned char* sorted = nullptr;
    std::uint64_t* scomp = nullptr;
    std::uint8_t* sstatus = nullptr;
    auto release = [&]() {
        dfree(keys_a); dfree(keys_b); dfree(pos_a); dfree(pos_b); dfree(temp);
        dfree(sorted); dfree(scomp); dfree(sstatus);
    };
    const unsigned end_bit = packed ? 56u : 64u;
    std::size_t temp_bytes = 0;
    hipError_t err = rocprim::radix_sort_pairs(nullptr, temp_bytes,
                                               static_cast<std::uint64_t*>(nullptr),
                                               static_cast<std::uint64_t*>(nullptr),
                                               static_cast<std::uint32_t*>(nullptr),
                                               static_cast<std::uint32_t*>(nullptr), n, 0, end_bit,
                                               stream);
    if (err == hipSuccess) err = dalloc(keys_a, n);
    if (err == hipSuccess) err = dalloc(keys_b, n);
    if (err == hipSuccess) err = dalloc(pos_a, n);
    if (err == hipSuccess) err = dalloc(pos_b, n);
    if (err == hipSuccess) err = hipMalloc(&temp, temp_bytes == 0 ? 1 : temp_bytes);
    if (err == hipSuccess) {
        if (packed) {
            hipLaunchKernelGGL(k_issue_keys<true>, dim3(blocks_for(n)), dim3(kThreads), 0, stream,
                               d_rec, n, keys_a, pos_a);
        } else {
            hipLaunchKernelGGL(k_issue_keys<false>, dim3(blocks_for(n)), dim3(kThreads), 0, stream,
                               d_rec, n, keys_a, pos_a);
        }
        err = hipGetLastError();
    }
    if (err == hipSuccess) {
        err = rocprim::radix_sort_pairs(temp, temp_bytes, keys_a, keys_b, pos_a, pos_b, n, 0,
                                        end_bit, stream);
    }
    // only the permutation is kept; the keys go before the copy is made
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    dfree(keys_a);
    dfree(keys_b);
    dfree(pos_a);
    dfree(temp);
    if (err == hipSuccess) err = hipMalloc(reinterpret_cast<void**>(&sorted), n * rec_bytes);
    if (err == hipSuccess) err = dalloc(scomp, n);
    if (err == hipSuccess && d_status != nullptr) err = dalloc(sstatus, n);
    if (err == hipSuccess) {
        if (packed) {
            hipLaunchKernelGGL(k_gather_records<hbf_record16>, dim3(blocks_for(n)), dim3(kThreads),
                               0, stream, static_cast<const hbf_record16*>(d_rec), pos_b, n,
                               reinterpret_cast<hbf_record16*>(sorted));
        } else {
            hipLaunchKernelGGL(k_gather_records<hbf_record32>, dim3(blocks_for(n)), dim3(kThreads),
                               0, stream, static_cast<const hbf_record32*>(d_rec), pos_b, n,
                               reinterpret_cast<hbf_record32*>(sorted));
        }
        err = hipGetLastError();
    }
    if (err != hipSuccess) {
        release();
        return HBFSIM_CUDA_ERROR;
    }
    const int st = run(sorted, scomp, sstatus);
    if (st != HBFSIM_OK) {
        (void)hipStreamSynchronize(stream);
        release();
        return st;
    }
    hipLaunchKernelGGL(k_scatter, dim3(blocks_for(n)), dim3(kThreads), 0, stream,
                       static_cast<const std::uint32_t*>(pos_b), n,
                       static_cast<const std::uint64_t*>(scomp),
                       static_cast<const std::uint8_t*>(sstatus), d_comp, d_status);
    err = hipGetLastError();
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    release();
    return err == hipSuccess ? HBFSIM_OK : HBFSIM_CUDA_ERROR;
}

}  // namespace hbfamd
