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
// geometry, engine defaults) is the media port of the MQSim adapter's
// admission (mqsim_online.cpp:291-376): at most the profile's queue_depth
// requests are in the device, a request that arrives while it is full waits
// in arrival order and enters when a completion frees a slot, and the engine
// times its pages issued at that admission time; a request's device
// completion is the ceiling in ns of its last page's.  Completions then pass
// the adapter's bandwidth cursor in completion order (ties in dispatch
// order).  Admission couples each request to earlier completions, which
// depend on the engine state the earlier requests left: the requests are
// taken in chunks of queue_depth, and a chunk's admission times are iterated
// to their fixed point, the engine state restored before each retry (device
// completions grow with admission times, so the iteration rises from
// admission = arrival to the event loop's times, one request at least per
// pass).  Latencies are bounded completion - arrival in ns.  Exit 64 on
// invalid arguments, 70 on other errors, as the reference.
#include "cli_json.hpp"
#include "profile.hpp"

#include "../../include/hbfsim_amd.h"

#include <algorithm>
#include <queue>
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

// Admission times of requests [c, e): a request enters at its arrival while
// fewer than `depth` requests are in the device, else at the later of its
// arrival and the earliest device completion among those in it (FIFO, one
// slot per completion).  `held` holds the device completions of the requests
// in the device before c; dev[c..e) the current estimates (an admission time
// stands for a completion not yet known: completions are never earlier).
std::vector<std::uint64_t> chunk_admissions(
    const std::priority_queue<std::uint64_t, std::vector<std::uint64_t>,
                              std::greater<std::uint64_t>>& held,
    std::uint64_t depth, const std::vector<std::uint64_t>& arrival, std::uint64_t c,
    std::uint64_t e, const std::vector<std::uint64_t>* dev)
{
    auto h = held;
    std::vector<std::uint64_t> adm(e - c);
    for (std::uint64_t i = c; i < e; ++i) {
        std::uint64_t a = arrival[i];
        if (h.size() >= depth) {
            a = std::max(a, h.top());
            h.pop();
        }
        adm[i - c] = a;
        h.push(dev != nullptr ? std::max((*dev)[i - c], a) : a);
    }
    return adm;
}

// Times the requests through the engine under queue-depth admission (see the
// file comment): per chunk of `depth` requests, admission times and device
// completions iterated to their fixed point, the engine state restored
// before every retry.  completion/status per record; device_ns per request.
int admit_and_time(hbfsim_context* ctx, std::uint64_t requests, std::uint64_t depth,
                   const std::vector<std::uint64_t>& arrival,
                   const std::vector<std::uint64_t>& last, std::vector<hbf_record32>& records,
                   std::vector<std::uint64_t>& completion, std::vector<std::uint8_t>& status,
                   std::vector<std::uint64_t>& device_ns)
{
    std::uint32_t channels = 0, planes = 0;
    int st = hbfsim_amd_get_geometry(ctx, &channels, &planes);
    if (st != HBFSIM_OK) {
        return st;
    }
    std::vector<std::uint64_t> busy(planes), tags(2ull * planes), cursor(channels);
    std::priority_queue<std::uint64_t, std::vector<std::uint64_t>, std::greater<std::uint64_t>>
        held;
    for (std::uint64_t c = 0; c < requests; c += depth) {
        const std::uint64_t e = std::min(requests, c + depth);
        const std::uint64_t r0 = c == 0 ? 0 : last[c - 1] + 1, r1 = last[e - 1] + 1;
        std::uint64_t seq = 0, burst = 0;
        st = hbfsim_amd_get_state(ctx, busy.data(), tags.data(), cursor.data(), &seq, &burst);
        if (st != HBFSIM_OK) {
            return st;
        }
        std::vector<std::uint64_t> adm = chunk_admissions(held, depth, arrival, c, e, nullptr);
        std::vector<std::uint64_t> dev(e - c);
        for (std::uint64_t pass = 0;; ++pass) {
            if (pass > 0) {
                st = hbfsim_amd_set_state(ctx, busy.data(), tags.data(), cursor.data(), seq, burst);
                if (st != HBFSIM_OK) {
                    return st;
                }
            }
            std::uint64_t r = r0;
            for (std::uint64_t i = c; i < e; ++i) {
                for (; r <= last[i]; ++r) {
                    records[r].issue_ps = adm[i - c] * 1000u;
                }
            }
            st = hbfsim_amd_run(ctx, records.data() + r0, r1 - r0, completion.data() + r0,
                                status.data() + r0, 0, nullptr);
            if (st != HBFSIM_OK) {
                return st;
            }
            r = r0;
            for (std::uint64_t i = c; i < e; ++i) {
                std::uint64_t done_ps = adm[i - c] * 1000u;
                for (; r <= last[i]; ++r) {
                    done_ps = std::max(done_ps, completion[r]);
                }
                dev[i - c] = (done_ps + 999) / 1000;
            }
            std::vector<std::uint64_t> next = chunk_admissions(held, depth, arrival, c, e, &dev);
            if (next == adm) {
                break;  // the times the engine ran with are the fixed point
            }
            if (pass > e - c) {
                return HBFSIM_INVALID_ARGUMENT;  // cannot happen: one request settles per pass
            }
            adm = std::move(next);
        }
        for (std::uint64_t i = c; i < e; ++i) {
            if (held.size() >= depth) {
                held.pop();
            }
            held.push(dev[i - c]);
            device_ns[i] = dev[i - c];
        }
    }
    return HBFSIM_OK;
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
        std::vector<std::uint64_t> arrival_ns;
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
            arrival_ns.push_back(arrival_ps / 1000);
        }
        const std::uint64_t depth = std::max<std::uint64_t>(1, prof.queue_depth);
        std::vector<std::uint64_t> completion(records.size());
        std::vector<std::uint8_t> status(records.size());
        std::vector<std::uint64_t> device_ns(o.requests);
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
                st = admit_and_time(ctx, o.requests, depth, arrival_ns, last, records,
                                    completion, status, device_ns);
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

        for (const std::uint8_t b : status) {
            if ((b & 3u) != HBFSIM_AMD_MODELED) {
                throw std::runtime_error("the engine did not model a benchmark request");
            }
        }
        // the adapter's completion callbacks, in completion order (ties in
        // dispatch order, which is request order): the bandwidth cursor
        std::vector<std::uint64_t> order(o.requests);
        for (std::uint64_t i = 0; i < o.requests; ++i) order[i] = i;
        std::sort(order.begin(), order.end(), [&](std::uint64_t a, std::uint64_t b) {
            return device_ns[a] != device_ns[b] ? device_ns[a] < device_ns[b] : a < b;
        });
        const std::uint64_t xfer_ns = static_cast<std::uint64_t>(
            (static_cast<unsigned __int128>(o.bytes) * 1000000000u +
             prof.aggregate_bandwidth_bytes_per_s - 1) /
            prof.aggregate_bandwidth_bytes_per_s);
        std::vector<std::uint64_t> bounded(o.requests);
        std::uint64_t cursor = 0;
        for (const std::uint64_t k : order) {
            cursor = std::max(cursor, arrival_ns[k]) + xfer_ns;
            bounded[k] = std::max(device_ns[k], cursor);
        }
        std::vector<std::uint64_t> latencies;
        latencies.reserve(o.requests);
        std::uint64_t modeled_end_ns = 0;
        unsigned __int128 latency_sum = 0;
        for (std::uint64_t i = 0; i < o.requests; ++i) {
            latencies.push_back(bounded[i] - arrival_ns[i]);
            latency_sum += bounded[i] - arrival_ns[i];
            modeled_end_ns = std::max(modeled_end_ns, bounded[i]);
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
           << "  \"queue_depth\": " << depth << ",\n"
           << "  \"queue_depth_applied\": true,\n"
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
