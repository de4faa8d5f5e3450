// gen.hip -- workload compiler: segments of sequential lines -> access records.
//
// A decode step that streams weights reads each selected tensor (or expert)
// front to back in fixed-size lines, spread round-robin over `issuers`
// concurrent wavefronts that each issue one line every `gap_ps`.  Record j of
// the step: segment s = j / lines, line k = j % lines,
//   addr = seg_base[s] + k * line_bytes, issue_ps = (j / issuers) * gap_ps.
// Records come out ordered by issue time, as the timing engine requires.
#include <hip/hip_runtime.h>

#include "engine.hpp"

#include <algorithm>

namespace hbfamd {
namespace {

__global__ __launch_bounds__(256) void k_gen_lines(hbf_record32* out, std::uint64_t n,
                                                   const std::uint64_t* seg_base,
                                                   std::uint64_t lines, std::uint32_t line_bytes,
                                                   std::uint64_t gap_ps, std::uint32_t issuers,
                                                   std::uint64_t flags)
{
    const std::uint64_t stride = static_cast<std::uint64_t>(gridDim.x) * blockDim.x;
    for (std::uint64_t j = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
         j < n; j += stride) {
        std::uint64_t s, k, slot;
        if (n <= 0xffffffffull) {  // 32-bit division when the batch allows
            const std::uint32_t j32 = static_cast<std::uint32_t>(j);
            const std::uint32_t l32 = static_cast<std::uint32_t>(lines);
            s = j32 / l32;
            k = j32 - static_cast<std::uint32_t>(s) * l32;
            slot = j32 / issuers;
        } else {
            s = j / lines;
            k = j - s * lines;
            slot = j / issuers;
        }
        uint4* p = reinterpret_cast<uint4*>(out + j);
        const std::uint64_t addr = seg_base[s] + k * line_bytes;
        const std::uint64_t issue = slot * gap_ps;
        p[0] = make_uint4(static_cast<std::uint32_t>(addr), static_cast<std::uint32_t>(addr >> 32),
                          line_bytes, 0u);
        p[1] = make_uint4(static_cast<std::uint32_t>(issue),
                          static_cast<std::uint32_t>(issue >> 32),
                          static_cast<std::uint32_t>(flags),
                          static_cast<std::uint32_t>(flags >> 32));
    }
}

// Spans of consecutive lines, each with its own length and operation: span
// s covers records [first[s], first[s + 1]) of the step and reads (op 0) or
// writes (op 1) lines base[s] + k * line_bytes.  One workgroup walks a span;
// issue times follow the record index as above.
__global__ __launch_bounds__(256) void k_gen_spans(hbf_record32* out,
                                                   const std::uint64_t* base,
                                                   const std::uint64_t* first,
                                                   const std::uint32_t* op, std::uint64_t nspan,
                                                   std::uint32_t line_bytes, std::uint64_t gap_ps,
                                                   std::uint32_t issuers)
{
    for (std::uint64_t s = blockIdx.x; s < nspan; s += gridDim.x) {
        const std::uint64_t j0 = first[s];
        const std::uint64_t len = first[s + 1] - j0;
        const std::uint64_t b = base[s];
        const std::uint32_t o = op[s];
        for (std::uint64_t k = threadIdx.x; k < len; k += blockDim.x) {
            const std::uint64_t j = j0 + k;
            const std::uint64_t addr = b + k * line_bytes;
            const std::uint64_t issue = (j / issuers) * gap_ps;
            uint4* p = reinterpret_cast<uint4*>(out + j);
            p[0] = make_uint4(static_cast<std::uint32_t>(addr),
                              static_cast<std::uint32_t>(addr >> 32), line_bytes, 0u);
            p[1] = make_uint4(static_cast<std::uint32_t>(issue),
                              static_cast<std::uint32_t>(issue >> 32), o, 0u);
        }
    }
}

}  // namespace

int gen_spans(hbf_record32* d_records, std::size_t capacity, const std::uint64_t* d_base,
              const std::uint64_t* d_first, const std::uint32_t* d_op, std::size_t nspan,
              std::uint64_t total, std::uint32_t line_bytes, std::uint64_t gap_ps,
              std::uint32_t issuers, void* stream)
{
    if (d_records == nullptr || d_base == nullptr || d_first == nullptr || d_op == nullptr ||
        nspan == 0 || line_bytes == 0 || issuers == 0 || total > capacity ||
        (reinterpret_cast<std::uintptr_t>(d_records) & 15u) != 0) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    const unsigned blocks = static_cast<unsigned>(std::min<std::uint64_t>(nspan, 1u << 20));
    hipLaunchKernelGGL(k_gen_spans, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                       d_records, d_base, d_first, d_op, nspan, line_bytes, gap_ps, issuers);
    if (hipGetLastError() != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    return HBFSIM_OK;
}

int gen_segment_lines(hbf_record32* d_records, std::size_t capacity, const std::uint64_t* d_seg_base,
                      std::size_t nseg, std::uint64_t lines, std::uint32_t line_bytes,
                      std::uint64_t gap_ps, std::uint32_t issuers, std::uint64_t flags,
                      void* stream)
{
    if (d_records == nullptr || d_seg_base == nullptr || nseg == 0 || lines == 0 ||
        line_bytes == 0 || issuers == 0 ||
        (reinterpret_cast<std::uintptr_t>(d_records) & 15u) != 0) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    const unsigned __int128 total = static_cast<unsigned __int128>(nseg) * lines;
    if (total > capacity || lines > 0xffffffffull) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    const std::uint64_t n = static_cast<std::uint64_t>(total);
    const unsigned blocks =
        static_cast<unsigned>(std::min<std::uint64_t>((n + 255) / 256, 256ull * 64));
    hipLaunchKernelGGL(k_gen_lines, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                       d_records, n, d_seg_base, lines, line_bytes, gap_ps, issuers, flags);
    if (hipGetLastError() != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    return HBFSIM_OK;
}

}  // namespace hbfamd
