// profile.cpp -- HBF device profile loading and validation.
//
// Follows the reference loader's field list, defaults, rule order and
// messages (src/profile/profile.cpp:160-192, 238-468).
#include "profile.hpp"

#include "json_min.hpp"

#include <cmath>
#include <fstream>
#include <sstream>

namespace hbfamd {
namespace {

bool is_power_of_two(std::uint32_t v) { return v != 0 && (v & (v - 1)) == 0; }

void require_nonzero(std::uint32_t v, const char* field)
{
    if (v == 0) {
        throw profile_error(std::string(field) + " must be greater than zero");
    }
}

void parse_empirical(const json_min::value& doc, empirical_vmem& e)
{
    const json_min::value* found = doc.find("empirical_vmem");
    if (found == nullptr) {
        return;
    }
    const json_min::value& emp = *found;
    const json_min::value& curve = emp.at("read_curve");
    if (curve.kind != json_min::value::array_t || curve.a.size() != 6) {
        throw profile_error("empirical_vmem read_curve must contain exactly 6 points");
    }
    e.present = true;
    e.source_kind = emp.at("source_kind").as_string();
    e.source_sha256 = emp.at("source_sha256").as_string();
    e.source_capacity_bytes = emp.at("source_capacity_bytes").as_u64();
    e.quantile = emp.at("quantile").as_string();
    e.sample_count = emp.at("sample_count").as_u32();
    for (std::size_t i = 0; i < 6; ++i) {
        e.read_curve[i].pages = curve.a[i].at("pages").as_u32();
        e.read_curve[i].cumulative_ns = curve.a[i].at("cumulative_ns").as_u64();
        e.read_curve[i].p95_ns = curve.a[i].at("p95_ns").as_u64();
    }
    e.program_p50_ns = emp.at("program_p50_ns").as_u64();
    e.program_p95_ns = emp.at("program_p95_ns").as_u64();
}

}  // namespace

bool parse_allocation_scheme(const std::string& text, std::uint32_t order[4])
{
    if (text.size() != 4) {
        return false;
    }
    std::uint32_t seen = 0;
    for (int i = 0; i < 4; ++i) {
        std::uint32_t axis;
        switch (text[i]) {
        case 'C': axis = 0; break;
        case 'W': axis = 1; break;
        case 'D': axis = 2; break;
        case 'P': axis = 3; break;
        default: return false;
        }
        if (seen & (1u << axis)) {
            return false;
        }
        seen |= 1u << axis;
        order[i] = axis;
    }
    return true;
}

std::uint64_t blocks_per_plane(const profile& p, std::uint32_t chips)
{
    if (p.page_bytes == 0 || p.channels == 0 || chips == 0 ||
        p.dies_per_channel == 0 || p.planes_per_die == 0 || p.pages_per_block == 0) {
        throw profile_error(
            "capacity geometry must contain an integral number of blocks per plane");
    }
    const unsigned __int128 denominator =
        static_cast<unsigned __int128>(p.page_bytes) * p.channels * chips *
        p.dies_per_channel * p.planes_per_die * p.pages_per_block;
    if (denominator > UINT64_MAX ||
        p.capacity_bytes % static_cast<std::uint64_t>(denominator) != 0) {
        throw profile_error(
            "capacity geometry must contain an integral number of blocks per plane");
    }
    const std::uint64_t blocks = p.capacity_bytes / static_cast<std::uint64_t>(denominator);
    if (blocks == 0) {
        throw profile_error(
            "capacity geometry must contain an integral number of blocks per plane");
    }
    return blocks;
}

void validate_profile(const profile& p, std::uint32_t chips)
{
    if (p.capacity_bytes == 0) {
        throw profile_error("capacity_bytes must be greater than zero");
    }
    if (!is_power_of_two(p.page_bytes)) {
        throw profile_error("page_bytes must be a power of two");
    }
    if (p.page_bytes < 512) {
        throw profile_error("page_bytes must be at least 512 for MQSim sector alignment");
    }
    if (p.read_latency_ns == 0) {
        throw profile_error("read_latency_ns must be greater than zero");
    }
    if (p.program_latency_ns == 0) {
        throw profile_error("program_latency_ns must be greater than zero");
    }
    require_nonzero(p.channels, "channels");
    require_nonzero(p.dies_per_channel, "dies_per_channel");
    require_nonzero(p.planes_per_die, "planes_per_die");
    require_nonzero(p.pages_per_block, "pages_per_block");
    require_nonzero(p.channel_width_bits, "channel_width_bits");
    require_nonzero(p.channel_transfer_rate_mtps, "channel_transfer_rate_mtps");
    require_nonzero(p.queue_depth, "queue_depth");
    if (p.aggregate_bandwidth_bytes_per_s == 0) {
        throw profile_error("aggregate_bandwidth_bytes_per_s must be greater than zero");
    }
    if (p.hbm_cache_bytes > p.capacity_bytes) {
        throw profile_error("hbm_cache_bytes must not exceed capacity_bytes");
    }
    if (!std::isfinite(p.reference_sample_rate) || p.reference_sample_rate < 0.0 ||
        p.reference_sample_rate > 1.0) {
        throw profile_error("reference_sample_rate must be in [0, 1]");
    }
    require_nonzero(p.time_scale, "time_scale");
    (void)blocks_per_plane(p, chips);
    for (int i = 0; i < 4; ++i) {
        if (p.page_read_latency_ns[i] == 0 || p.page_program_latency_ns[i] == 0) {
            throw profile_error(
                "per-level page read/program latencies must be greater than zero");
        }
    }
    if (!p.empirical.present) {
        return;
    }
    const empirical_vmem& e = p.empirical;
    if (p.page_bytes != 4096) {
        throw profile_error("empirical_vmem requires page_bytes == 4096");
    }
    bool valid_sha = e.source_sha256.size() == 64;
    for (char c : e.source_sha256) {
        valid_sha = valid_sha && ((c >= '0' && c <= '9') || (c >= 'a' && c <= 'f'));
    }
    if (!valid_sha) {
        throw profile_error("empirical_vmem source_sha256 must be lowercase hexadecimal SHA256");
    }
    if (e.source_kind.empty()) {
        throw profile_error("empirical_vmem source_kind must not be empty");
    }
    if (e.source_capacity_bytes == 0) {
        throw profile_error("empirical_vmem source_capacity_bytes must be greater than zero");
    }
    if (e.quantile != "p50") {
        throw profile_error("empirical_vmem quantile must be p50");
    }
    if (e.sample_count == 0) {
        throw profile_error("empirical_vmem sample_count must be greater than zero");
    }
    for (std::size_t i = 0; i < 6; ++i) {
        const empirical_point& pt = e.read_curve[i];
        if (i != 0 && pt.pages <= e.read_curve[i - 1].pages) {
            throw profile_error("empirical_vmem pages must be strictly increasing");
        }
        if (pt.cumulative_ns == 0 ||
            (i != 0 && pt.cumulative_ns <= e.read_curve[i - 1].cumulative_ns)) {
            throw profile_error("empirical_vmem P50 latency must be strictly increasing");
        }
        if (pt.p95_ns < pt.cumulative_ns) {
            throw profile_error("empirical_vmem P95 latency must not be below P50");
        }
    }
    if (e.read_curve[5].pages > 1023) {
        throw profile_error("empirical_vmem final page must not exceed 1023");
    }
    if (e.program_p50_ns == 0) {
        throw profile_error("empirical_vmem program P50 must be greater than zero");
    }
    if (e.program_p95_ns < e.program_p50_ns) {
        throw profile_error("empirical_vmem program P95 must not be below P50");
    }
}

profile load_profile(const std::string& path)
{
    std::ifstream input(path);
    if (!input) {
        throw profile_error("could not open profile: " + path);
    }
    std::stringstream buffer;
    buffer << input.rdbuf();
    profile p;
    try {
        const json_min::value doc = json_min::parse(buffer.str());
        p.name = doc.at("name").as_string();
        p.capacity_bytes = doc.at("capacity_bytes").as_u64();
        p.page_bytes = doc.at("page_bytes").as_u32();
        p.read_latency_ns = doc.at("read_latency_ns").as_u64();
        p.program_latency_ns = doc.at("program_latency_ns").as_u64();
        p.channels = doc.at("channels").as_u32();
        p.dies_per_channel = doc.at("dies_per_channel").as_u32();
        p.planes_per_die = doc.at("planes_per_die").as_u32();
        p.pages_per_block = doc.at("pages_per_block").as_u32();
        p.channel_width_bits = doc.at("channel_width_bits").as_u32();
        p.channel_transfer_rate_mtps = doc.at("channel_transfer_rate_mtps").as_u32();
        p.queue_depth = doc.at("queue_depth").as_u32();
        p.aggregate_bandwidth_bytes_per_s = doc.at("aggregate_bandwidth_bytes_per_s").as_u64();
        p.hbm_cache_bytes = doc.at("hbm_cache_bytes").as_u64();
        p.reference_sample_rate = doc.at("reference_sample_rate").as_double();
        p.reference_warmup_requests = doc.at("reference_warmup_requests").as_u32();
        p.time_scale = doc.at("time_scale").as_u32();
        p.timing_tolerance_ns = doc.at("timing_tolerance_ns").as_u64();
        if (doc.contains("nand_technology")) {
            const std::string& t = doc.at("nand_technology").as_string();
            if (t != "SLC" && t != "MLC" && t != "TLC" && t != "QLC") {
                throw profile_error("nand_technology must be one of SLC, MLC, TLC, QLC");
            }
            p.nand_technology = t;
        }
        if (doc.contains("plane_allocation_scheme")) {
            const std::string& s = doc.at("plane_allocation_scheme").as_string();
            if (!parse_allocation_scheme(s, p.axis_order)) {
                throw profile_error(
                    "plane_allocation_scheme must be one of the 24 channel/way/die/plane "
                    "orderings, e.g. CWDP");
            }
            p.plane_allocation_scheme = s;
        }
        parse_empirical(doc, p.empirical);
        static const char* read_keys[4] = {"page_read_latency_lsb_ns", "page_read_latency_csb_ns",
                                           "page_read_latency_msb_ns", "page_read_latency_tsb_ns"};
        static const char* prog_keys[4] = {
            "page_program_latency_lsb_ns", "page_program_latency_csb_ns",
            "page_program_latency_msb_ns", "page_program_latency_tsb_ns"};
        for (int i = 0; i < 4; ++i) {
            p.page_read_latency_ns[i] = doc.contains(read_keys[i])
                                            ? doc.at(read_keys[i]).as_u64()
                                            : p.read_latency_ns;
            p.page_program_latency_ns[i] = doc.contains(prog_keys[i])
                                               ? doc.at(prog_keys[i]).as_u64()
                                               : p.program_latency_ns;
        }
    } catch (const profile_error&) {
        throw;
    } catch (const json_min::error& e) {
        throw profile_error(std::string("invalid profile JSON: ") + e.what());
    }
    validate_profile(p);
    return p;
}

}  // namespace hbfamd
