// link.hpp -- host interface of the UCIe Streaming / AoU link kernel.
#pragma once

#include "../../include/hbfsim_amd.h"

#include <cstddef>
#include <cstdint>

namespace hbfamd {

// hbfsim_amd_link_run (link.hip).  Synchronises `stream`.
// hbfsim_amd_link_run_traced with d_flits null and flit_limit 0.
int link_run(const hbfsim_amd_link_profile& profile, const std::uint64_t* d_first,
             std::uint32_t links, const std::uint64_t* d_ready, const std::uint8_t* d_direction,
             std::size_t n, std::uint64_t* d_delivered, hbfsim_amd_link_counters* d_counters,
             void* stream, hbfsim_amd_link_flit* d_flits = nullptr, std::uint32_t flit_limit = 0);

}  // namespace hbfamd
