// media_bench.cpp -- hbf_media_bench, the counterpart of the reference's
// hbf_mqsim_bench (benchmarks/mqsim/hbf_mqsim_bench.cpp:24-368) with this
// engine's device model in place of MQSim: the same options, the same
// workload (sequential slots, or splitmix64-drawn slots for
// --pattern random, arrivals index * gap, alternating operations for
// --operation mixed) and the same JSON report, keys sorted as
// nlohmann::json::dump(2) prints them.
//
//   hbf_media_bench --profile FILE [--requests N] [--bytes N]
//                   [--operation read|write|mixed] [--arrival-gap-ns N]
//                   [--capacity-bytes N] [--pattern sequential|random] [--seed N]
//
// Every request is split at page boundaries into records of one range that
// covers the benchmark capacity; the GPU engine (HBF model, profile
// geometry, engine defaults) times them, and a request completes with its
// last page.  Latencies are completion - arrival in ns (ceiling of the
// engine's picoseconds).  The engine's device accepts every request at its
// arrival: the MQSim adapter's queue-depth admission (mqsim_online.cpp:
// 291-376) couples each request to earlier completions and is not applied,
// which the report states in "queue_depth_applied".  Exit 64 on invalid
// arguments, 70 on other errors, as the reference.
#include "cli_json.hpp"
#include "profile.hpp"

#include "../../include/hbfsim_amd.h"

#include <algorithm>
#include <charconv>
#include <chrono>
#include <cstdint>
#include <filesystem>
#include <iostream>
#include <limits>
#include <sstream>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

#include <unistd.h>

namespace {

constexpr std::uint64_t kDefaultCacheCapacity = 64ull * 1024 * 1024;
constexpr std::uint64_t kDefaultBlocksPerPlane = 16;
constexpr std::uint64_t kRangeBase = 0x4000'0000'0000ull;

struct options {
    std::string profile_path;
    std::uint64_t requests{1024};
    std::uint32_t bytes{16384};
    std::string operation{"read"};
    std::uint64_t arrival_gap_ns{0};
    std::uint64_t capacity_bytes{0};
    std::string pattern{"sequential"};
    std::uint64_t seed{0};
};

[[noreturn]] void usage_error(const std::string& message)
{
    throw std::invalid_argument(
        message +
        "\nusage: hbf_media_bench --profile FILE [--requests N] [--bytes N] "
        "[--operation read|write|mixed] [--arrival-gap-ns N] [--capacity-bytes N] "
        "[--pattern sequential|random] [--seed N]");
}

std::uint64_t parse_u64(std::string_view text, std::string_view option)
{
    std::uint64_t value = 0;
    const auto r = std::from_chars(text.data(), text.data() + text.size(), value);
    if (r.ec != std::errc{} || r.ptr != text.data() + text.size()) {
        usage_error("invalid value for " + std::string(option));
    }
    return value;
}

options parse_options(int argc, char** argv)
{
    options o;
    for (int i = 1; i < argc; ++i) {
        const std::string_view opt{argv[i]};
        if (i + 1 >= argc) {
            usage_error("missing value for " + std::string(opt));
        }
        const std::string_view v{argv[++i]};
        if (opt == "--profile") {
            o.profile_path = v;
        } else if (opt == "--requests") {
            o.requests = parse_u64(v, opt);
        } else if (opt == "--bytes") {
            const std::uint64_t b = parse_u64(v, opt);
            if (b > std::numeric_limits<std::uint32_t>::max()) {
                usage_error("--bytes exceeds the request ABI limit");
            }
            o.bytes = static_cast<std::uint32_t>(b);
        } else if (opt == "--operation") {
            o.operation = v;
        } else if (opt == "--arrival-gap-ns") {
            o.arrival_gap_ns = parse_u64(v, opt);
        } else if (opt == "--capacity-bytes") {
            o.capacity_bytes = parse_u64(v, opt);
        } else if (opt == "--pattern") {
            o.pattern = v;
        } else if (opt == "--seed") {
            o.seed = parse_u64(v, opt);
        } else {
            usage_error("unknown option " + std::string(opt));
        }
    }
    if (o.profile_path.empty()) {
        usage_error("--profile is required");
    }
    if (o.requests == 0) {
        usage_error("--requests must be non-zero");
    }
    if (o.bytes == 0 || o.bytes % 512 != 0) {
        usage_error("--bytes must be a non-zero multiple of 512");
    }
    if (o.operation != "read" && o.operation != "write" && o.operation != "mixed") {
        usage_error("--operation must be read, write, or mixed");
    }
    if (o.pattern != "sequential" && o.pattern != "random") {
        usage_error("--pattern must be sequential or random");
    }
    if (o.capacity_bytes != 0 && o.capacity_bytes < o.bytes) {
        usage_error("--capacity-bytes must fit one request");
    }
    if (o.requests > 1 &&
        o.arrival_gap_ns > std::numeric_limits<std::uint64_t>::max() / (o.requests - 1)) {
        usage_error("benchmark arrival timeline overflows");
    }
    return o;
}

bool is_write(const options& o, std::uint64_t index)
{
    return o.operation == "write" || (o.operation == "mixed" && index % 2 != 0);
}

// splitmix64 (the published generator); draws each request's slot for
// --pattern random from the whole benchmark capacity
std::uint64_t splitmix64(std::uint64_t& state)
{
    state += 0x9e3779b97f4a7c15ull;
    std::uint64_t z = state;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

std::uint64_t percentile(const std::vector<std::uint64_t>& sorted, std::uint64_t percent)
{
    const std::uint64_t rank = (percent * sorted.size() + 99) / 100;
    return sorted[std::max<std::uint64_t>(1, rank) - 1];
}

std::uint64_t capacity_for_blocks(const hbfamd::profile& p, std::uint64_t blocks)
{
    const unsigned __int128 c = static_cast<unsigned __int128>(p.page_bytes) * p.pages_per_block *
                                p.planes_per_die * p.dies_per_channel * p.channels * blocks;
    if (c > std::numeric_limits<std::uint64_t>::max()) {
        throw std::overflow_error("benchmark profile geometry exceeds uint64 capacity");
    }
    return static_cast<std::uint64_t>(c);
}

void check(int status, const char* what)
{
    if (status != HBFSIM_OK) {
        throw std::runtime_error(std::string(what) + ": " + hbfsim_vllm_status_string(status));
    }
}

}  // namespace

int main(int argc, char** argv)
{
    using cli_json::quote;
    using cli_json::real;
    try {
        const options o = parse_options(argc, argv);
        hbfamd::profile prof = hbfamd::load_profile(o.profile_path);
        prof.capacity_bytes = o.capacity_bytes == 0
                                  ? std::min(prof.capacity_bytes,
                                             capacity_for_blocks(prof, kDefaultBlocksPerPlane))
                                  : o.capacity_bytes;
        prof.hbm_cache_bytes = std::min(prof.capacity_bytes, kDefaultCacheCapacity);
        hbfamd::validate_profile(prof);
        const std::uint64_t blocks = hbfamd::blocks_per_plane(prof);
        if (o.operation != "read" && blocks <= 10) {
            usage_error("write workloads require more than 10 blocks per plane; "
                        "increase --capacity-bytes");
        }
        // the workload: requests split at page boundaries into records
        const std::uint64_t slots = prof.capacity_bytes / o.bytes;
        const std::uint64_t page = prof.page_bytes;
        std::vector<hbf_record32> records;
        std::vector<std::uint64_t> last;  // each request's last record
        std::uint64_t state = o.seed;
        for (std::uint64_t i = 0; i < o.requests; ++i) {
            const std::uint64_t slot = o.pattern == "random" ? splitmix64(state) % slots
                                                             : i % slots;
            const std::uint64_t arrival_ps = static_cast<std::uint64_t>(
                static_cast<unsigned __int128>(i) * o.arrival_gap_ns * 1000u);
            std::uint64_t addr = slot * o.bytes;
            std::uint64_t left = o.bytes;
            while (left != 0) {
                const std::uint64_t piece = std::min(left, page - addr % page);
                records.push_back({kRangeBase + addr, piece, arrival_ps, is_write(o, i) ? 1u : 0u});
                addr += piece;
                left -= piece;
            }
            last.push_back(records.size() - 1);
        }
        std::vector<std::uint64_t> completion(records.size());
        std::vector<std::uint8_t> status(records.size());
        const std::filesystem::path dir = std::filesystem::temp_directory_path() /
                                          ("hbf-media-bench-" + std::to_string(::getpid()));
        std::filesystem::create_directories(dir);
        const std::string dir_s = dir.string();
        const auto wall_start = std::chrono::steady_clock::now();
        {
            const hbfsim_options co{o.profile_path.c_str(), dir_s.c_str(), HBFSIM_MODEL_FAST, 64,
                                    1000000000ull};
            hbfsim_context* ctx = nullptr;
            check(hbfsim_context_create(&co, &ctx), "context");
            const hbfsim_range_options ro{HBFSIM_RANGE_MODE_TIMING, HBFSIM_RANGE_READ_WRITE,
                                          HBFSIM_CACHE_POLICY_NONE, 0};
            int st = hbfsim_register_device(ctx, reinterpret_cast<void*>(kRangeBase),
                                            prof.capacity_bytes, &ro);
            if (st == HBFSIM_OK) {
                st = hbfsim_amd_run(ctx, records.data(), records.size(), completion.data(),
                                    status.data(), 0, nullptr);
            }
            hbfsim_context_destroy(ctx);
            check(st, "engine run");
        }
        const auto wall_ns = static_cast<std::uint64_t>(
            std::chrono::duration_cast<std::chrono::nanoseconds>(
                std::chrono::steady_clock::now() - wall_start)
                .count());
        std::error_code ec;
        std::filesystem::remove_all(dir, ec);

        std::vector<std::uint64_t> latencies;
        latencies.reserve(o.requests);
        std::uint64_t modeled_end_ns = 0;
        unsigned __int128 latency_sum = 0;
        std::size_t r = 0;
        for (std::uint64_t i = 0; i < o.requests; ++i) {
            std::uint64_t done_ps = 0;
            for (; r <= last[i]; ++r) {
                if ((status[r] & 3u) != HBFSIM_AMD_MODELED) {
                    throw std::runtime_error("the engine did not model a benchmark request");
                }
                done_ps = std::max(done_ps, completion[r]);
            }
            const std::uint64_t done_ns = (done_ps + 999) / 1000;
            const std::uint64_t arrival_ns = i * o.arrival_gap_ns;
            latencies.push_back(done_ns - arrival_ns);
            latency_sum += done_ns - arrival_ns;
            modeled_end_ns = std::max(modeled_end_ns, done_ns);
        }
        std::sort(latencies.begin(), latencies.end());
        const long double total_bytes =
            static_cast<long double>(o.requests) * static_cast<long double>(o.bytes);
        const std::uint64_t average =
            static_cast<std::uint64_t>(latency_sum / static_cast<unsigned __int128>(o.requests));
        const double bandwidth =
            static_cast<double>(total_bytes * 1.0e9L / static_cast<long double>(modeled_end_ns));
        const double rate = static_cast<double>(static_cast<long double>(o.requests) * 1.0e9L /
                                                static_cast<long double>(std::max<std::uint64_t>(wall_ns, 1)));
        std::ostringstream os;
        os << "{\n"
           << "  \"effective_profile\": {\n"
           << "    \"aggregate_bandwidth_bytes_per_s\": " << prof.aggregate_bandwidth_bytes_per_s
           << ",\n"
           << "    \"blocks_per_plane\": " << blocks << ",\n"
           << "    \"capacity_bytes\": " << prof.capacity_bytes << ",\n"
           << "    \"channels\": " << prof.channels << ",\n"
           << "    \"hbm_cache_bytes\": " << prof.hbm_cache_bytes << ",\n"
           << "    \"nand_technology\": " << quote(prof.nand_technology) << ",\n"
           << "    \"plane_allocation_scheme\": " << quote(prof.plane_allocation_scheme) << ",\n"
           << "    \"program_latency_ns\": " << prof.program_latency_ns << ",\n"
           << "    \"read_latency_ns\": " << prof.read_latency_ns << "\n"
           << "  },\n"
           << "  \"engine\": \"hbf-amd-media-only\",\n"
           << "  \"latency_ns\": {\n"
           << "    \"average\": " << average << ",\n"
           << "    \"p50\": " << percentile(latencies, 50) << ",\n"
           << "    \"p99\": " << percentile(latencies, 99) << "\n"
           << "  },\n"
           << "  \"modeled_bandwidth_bytes_per_s\": " << real(bandwidth) << ",\n"
           << "  \"profile\": " << quote(prof.name) << ",\n"
           << "  \"queue_depth_applied\": false,\n"
           << "  \"requests\": {\n"
           << "    \"completed\": " << o.requests << ",\n"
           << "    \"submitted\": " << o.requests << "\n"
           << "  },\n"
           << "  \"schema_version\": 1,\n"
           << "  \"simulator_requests_per_s\": " << real(rate) << ",\n"
           << "  \"timing_ns\": {\n"
           << "    \"modeled\": " << modeled_end_ns << ",\n"
           << "    \"wall\": " << wall_ns << "\n"
           << "  },\n"
           << "  \"workload\": {\n"
           << "    \"arrival_gap_ns\": " << o.arrival_gap_ns << ",\n"
           << "    \"bytes_per_request\": " << o.bytes << ",\n"
           << "    \"operation\": " << quote(o.operation) << ",\n"
           << "    \"pattern\": " << quote(o.pattern) << ",\n"
           << "    \"requests\": " << o.requests << ",\n"
           << "    \"seed\": " << o.seed << "\n"
           << "  }\n"
           << "}\n";
        std::cout << os.str();
        return 0;
    } catch (const std::invalid_argument& e) {
        std::cerr << "hbf_media_bench: " << e.what() << '\n';
        return 64;
    } catch (const std::exception& e) {
        std::cerr << "hbf_media_bench: " << e.what() << '\n';
        return 70;
    }
}
