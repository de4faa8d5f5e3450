// profile.hpp -- HBF device profile: fields, loading and validation.
//
// Same JSON document and validation rules as the reference loader
// (include/hbfsim/profile.hpp:79-110, src/profile/profile.cpp:238-468),
// including its error messages, so a profile that loads there loads here and
// a rejected one is rejected with the same text.
#pragma once

#include <array>
#include <cstdint>
#include <stdexcept>
#include <string>

namespace hbfamd {

struct profile_error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

struct empirical_point {
    std::uint32_t pages;
    std::uint64_t cumulative_ns;
    std::uint64_t p95_ns;
};

struct empirical_vmem {
    bool present{false};
    std::string source_kind;
    std::string source_sha256;
    std::uint64_t source_capacity_bytes{0};
    std::string quantile;
    std::uint32_t sample_count{0};
    std::array<empirical_point, 6> read_curve{};
    std::uint64_t program_p50_ns{0};
    std::uint64_t program_p95_ns{0};
};

struct profile {
    std::string name;
    std::uint64_t capacity_bytes{0};
    std::uint32_t page_bytes{0};
    std::uint64_t read_latency_ns{0};
    std::uint64_t program_latency_ns{0};
    std::uint32_t channels{0};
    std::uint32_t dies_per_channel{0};
    std::uint32_t planes_per_die{0};
    std::uint32_t pages_per_block{0};
    std::uint32_t channel_width_bits{0};
    std::uint32_t channel_transfer_rate_mtps{0};
    std::uint32_t queue_depth{0};
    std::uint64_t aggregate_bandwidth_bytes_per_s{0};
    std::uint64_t hbm_cache_bytes{0};
    double reference_sample_rate{0.0};
    std::uint32_t reference_warmup_requests{0};
    std::uint32_t time_scale{0};
    std::uint64_t timing_tolerance_ns{0};
    std::string nand_technology{"SLC"};
    std::uint64_t page_read_latency_ns[4]{};     // LSB, CSB, MSB, TSB
    std::uint64_t page_program_latency_ns[4]{};
    std::string plane_allocation_scheme{"CWDP"};
    std::uint32_t axis_order[4]{0, 1, 2, 3};    // fastest first: C W D P
    empirical_vmem empirical;
};

// profile.cpp:238-320; throws profile_error with the reference's messages.
profile load_profile(const std::string& path);
// profile.cpp:327-468 (legacy geometry: one chip per channel)
void validate_profile(const profile& p, std::uint32_t chips_per_channel = 1);
// profile.cpp:160-192
std::uint64_t blocks_per_plane(const profile& p, std::uint32_t chips_per_channel = 1);
// profile.cpp:100-136: "CWDP" etc. -> fastest-first axis ids (C0 W1 D2 P3)
bool parse_allocation_scheme(const std::string& text, std::uint32_t order[4]);

}  // namespace hbfamd
