// admission.hip -- the MQSim adapter's queue-depth admission and bandwidth
// cursor (src/mqsim_adapter/mqsim_online.cpp:291-376) on the GPU, over a
// media port that completes every request one fixed latency after it is
// handed over.
//
// The adapter hands a request to the device when fewer than queue_depth are
// in it, else queues it (FIFO) until a completion frees a slot.  With one
// latency L and arrivals in order, the device completes requests in
// admission order, so the slot request i waits for is that of request
// i - queue_depth: admission_i = max(arrival_i, device_{i - depth}) and
// device_i = admission_i + L, the interleaved chains of k identical servers
// (media_servers, servers.hip).  Completions reach the callback in index
// order, so the bandwidth cursor
//   cursor_i = max(cursor_{i-1}, arrival_i) + x_i,  x_i = ceil(bytes_i 1e9 / bw)
// is a prefix scan of the maps c -> max(c + x_i, arrival_i + x_i) under
// (max,+) composition, and the bounded completion is max(device_i, cursor_i).
#include <hip/hip_runtime.h>

#include <rocprim/device/device_scan.hpp>

#include "engine.hpp"

#include <cstdint>

namespace hbfamd {
namespace {

// c -> max(c + a, b): the cursor map of one request, or of a run of them
struct CursorMap {
    std::uint64_t a, b;
};

__host__ __device__ inline std::uint64_t sat_add(std::uint64_t x, std::uint64_t y)
{
    return x > ~0ull - y ? ~0ull : x + y;
}

// first p, then q (saturating at 2^64 - 1, which the output pass refuses)
struct Compose {
    __host__ __device__ CursorMap operator()(const CursorMap& p, const CursorMap& q) const
    {
        const std::uint64_t pb = sat_add(p.b, q.a);
        return CursorMap{sat_add(p.a, q.a), pb > q.b ? pb : q.b};
    }
};

__global__ __launch_bounds__(256) void k_adm_maps(const std::uint64_t* arrival,
                                                  const std::uint64_t* bytes, std::uint64_t n,
                                                  std::uint64_t bandwidth, CursorMap* maps)
{
    const std::uint64_t i = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) {
        return;
    }
    // mqsim_online.cpp:326-330: transfer = ceil(bytes * 1e9 / bandwidth)
    const unsigned __int128 t =
        (static_cast<unsigned __int128>(bytes[i]) * 1000000000ull + bandwidth - 1) / bandwidth;
    const std::uint64_t x = t > ~0ull ? ~0ull : static_cast<std::uint64_t>(t);
    maps[i] = CursorMap{x, sat_add(arrival[i], x)};
}

__global__ __launch_bounds__(256) void k_adm_out(const std::uint64_t* device, const CursorMap* maps,
                                                 std::uint64_t n, std::uint64_t latency,
                                                 std::uint64_t* admission,
                                                 std::uint64_t* completion, int* bad)
{
    const std::uint64_t i = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) {
        return;
    }
    // the cursor starts at 0 and every arrival is >= 0, so cursor_i = b
    const std::uint64_t cursor = maps[i].b;
    if (cursor == ~0ull) {
        *bad = 1;
    }
    const std::uint64_t dev = device[i];
    if (admission != nullptr) {
        admission[i] = dev - latency;
    }
    completion[i] = dev > cursor ? dev : cursor;
}

}  // namespace

int mqsim_admission(const std::uint64_t* d_arrival, const std::uint64_t* d_bytes, std::size_t n,
                    std::uint32_t queue_depth, std::uint64_t latency_ns,
                    std::uint64_t bandwidth, std::uint64_t* d_admission,
                    std::uint64_t* d_completion, void* stream_ptr)
{
    if (bandwidth == 0) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    if (n == 0) {
        return HBFSIM_OK;
    }
    if (d_arrival == nullptr || d_bytes == nullptr || d_completion == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    std::uint64_t* device = nullptr;
    CursorMap* maps = nullptr;
    int* bad = nullptr;
    void* temp = nullptr;
    std::size_t temp_bytes = 0;
    int h_bad = 0;
    hipError_t err = hipMalloc(reinterpret_cast<void**>(&device), n * sizeof(std::uint64_t));
    if (err == hipSuccess) err = hipMalloc(reinterpret_cast<void**>(&maps), n * sizeof(CursorMap));
    if (err == hipSuccess) err = hipMalloc(reinterpret_cast<void**>(&bad), sizeof(int));
    if (err == hipSuccess) err = hipMemsetAsync(bad, 0, sizeof(int), stream);
    if (err == hipSuccess) {
        err = rocprim::inclusive_scan(nullptr, temp_bytes, maps, maps, n, Compose{}, stream);
    }
    if (err == hipSuccess) err = hipMalloc(&temp, temp_bytes);
    int st = err == hipSuccess ? HBFSIM_OK : HBFSIM_CUDA_ERROR;
    // admission: queue_depth identical servers of latency L (max(1, depth))
    if (st == HBFSIM_OK) {
        st = media_servers(d_arrival, n, queue_depth == 0 ? 1 : queue_depth, latency_ns, device,
                           stream);
    }
    if (st == HBFSIM_OK) {
        const dim3 grid(static_cast<unsigned>((n + 255) / 256));
        hipLaunchKernelGGL(k_adm_maps, grid, dim3(256), 0, stream, d_arrival, d_bytes,
                           static_cast<std::uint64_t>(n), bandwidth, maps);
        err = hipGetLastError();
        if (err == hipSuccess) {
            err = rocprim::inclusive_scan(temp, temp_bytes, maps, maps, n, Compose{}, stream);
        }
        if (err == hipSuccess) {
            hipLaunchKernelGGL(k_adm_out, grid, dim3(256), 0, stream, device, maps,
                               static_cast<std::uint64_t>(n), latency_ns, d_admission,
                               d_completion, bad);
            err = hipGetLastError();
        }
        if (err == hipSuccess)
            err = hipMemcpyAsync(&h_bad, bad, sizeof(int), hipMemcpyDeviceToHost, stream);
        if (err == hipSuccess) err = hipStreamSynchronize(stream);
        st = err == hipSuccess ? HBFSIM_OK : HBFSIM_CUDA_ERROR;
    }
    (void)hipFree(device);
    (void)hipFree(maps);
    (void)hipFree(bad);
    (void)hipFree(temp);
    if (st != HBFSIM_OK) {
        return st;
    }
    return h_bad != 0 ? HBFSIM_INVALID_ARGUMENT : HBFSIM_OK;
}

}  // namespace hbfamd
