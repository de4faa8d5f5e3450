// trace_timing.cpp -- drop-in for the reference's hbf_trace_timing CLI
// (benchmarks/replay/hbf_trace_timing.cpp:76-269).
//
//   hbf_trace_timing --profile FILE --events JSONL --mode fast|hybrid|mqsim
//
// Ordered blocking replay of expert-miss events: every event is split into
// page requests; in fast mode each page adds max(base, transfer) to the
// demand clock and fast_service_ns to the modeled service (base = tR for
// reads, tPROG for writes; transfer = ceil(page * 1e9 / aggregate)).  All
// pages of one event have the same cost, so an event contributes
// pages * cost in one saturating step -- the replay is parse-bound, and this
// is host code that streams the events.  In hybrid mode the library's GPU
// HybridSampler (hbfsim_amd_sampler_reference, calibrator.cpp:83-96) picks
// the requests the reference sends to its detailed engine, MQSim
// (hbf_trace_timing.cpp:196-213).  MQSim is not part of this build; the
// library's engine stands in for it: a picked page request arrives at the
// demand clock, the engine times it on the GPU (per-plane tR / tPROG with
// the page register, the channel cursor, its state carried from one picked
// request to the next), and, as after an MQSim completion, the clock moves to
// its completion (ns, rounded up) and the modeled service grows by
// completion - arrival.  The report names that engine in "reference_timing".
// mqsim mode needs MQSim for every request: it exits 2.
//
// Output: the reference's JSON report, keys sorted and two-space indented as
// nlohmann::json::dump(2) prints it.  Exit 64 on invalid arguments or
// events (std::invalid_argument in the reference), 2 on other errors.
#include "cli_json.hpp"
#include "json_min.hpp"
#include "profile.hpp"

#include <hip/hip_runtime.h>

#include "../../include/hbfsim_amd.h"

#include <charconv>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <filesystem>
#include <fstream>
#include <iostream>
#include <limits>
#include <sstream>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

namespace {

struct usage : std::invalid_argument {
    using std::invalid_argument::invalid_argument;
};

struct options {
    std::string profile_path, events_path, mode;
};

[[noreturn]] void usage_error(const std::string& message)
{
    throw usage(message +
                "\nusage: hbf_trace_timing --profile FILE --events JSONL "
                "--mode fast|hybrid|mqsim");
}

options parse_options(int argc, char** argv)
{
    options o;
    for (int i = 1; i < argc; i += 2) {
        if (i + 1 >= argc) {
            usage_error("missing option value");
        }
        const std::string_view opt(argv[i]);
        if (opt == "--profile") {
            o.profile_path = argv[i + 1];
        } else if (opt == "--events") {
            o.events_path = argv[i + 1];
        } else if (opt == "--mode") {
            o.mode = argv[i + 1];
        } else {
            usage_error("unknown option " + std::string(opt));
        }
    }
    if (o.profile_path.empty() || o.events_path.empty() ||
        (o.mode != "fast" && o.mode != "hybrid" && o.mode != "mqsim")) {
        usage_error("all options are required and --mode must be valid");
    }
    return o;
}

// a + n * b, saturating: the same as n saturating additions of b.
std::uint64_t sat_add_n(std::uint64_t a, std::uint64_t n, std::uint64_t b)
{
    if (b != 0 && n > (std::numeric_limits<std::uint64_t>::max() - a) / b) {
        return std::numeric_limits<std::uint64_t>::max();
    }
    return a + n * b;
}

// hbf_trace_timing.cpp:76-89
std::uint64_t transfer_ns(std::uint64_t bytes, std::uint64_t bandwidth)
{
    if (bytes == 0 || bandwidth == 0) {
        throw std::invalid_argument("invalid fast transfer inputs");
    }
    const unsigned __int128 v =
        (static_cast<unsigned __int128>(bytes) * 1000000000ull + bandwidth - 1) / bandwidth;
    if (v > std::numeric_limits<std::uint64_t>::max()) {
        throw std::overflow_error("fast transfer time overflows");
    }
    return static_cast<std::uint64_t>(v);
}

// calibrator.cpp:33-65 (fast_service_ns): max(base, transfer) with the
// transfer computed through the same rounding.
std::uint64_t fast_service(std::uint64_t base, std::uint64_t bytes, std::uint64_t bandwidth)
{
    const std::uint64_t t = transfer_ns(bytes, bandwidth);
    return t > base ? t : base;
}

struct event {
    std::uint64_t logical_address;
    std::uint64_t bytes;
    std::uint32_t page_bytes;
    bool write;
};

std::uint64_t number(const json_min::value& v)
{
    if (!v.is_number()) {
        throw std::runtime_error("type_error: expected a number");
    }
    return v.as_u64();
}

// hbf_trace_timing.cpp:92-121
event parse_event(const json_min::value& e, std::uint64_t input_sequence)
{
    if (e.kind != json_min::value::object_t) {
        throw std::runtime_error("type_error: event is not an object");
    }
    const json_min::value* sv = e.find("schema_version");
    const json_min::value* sq = e.find("sequence");
    if ((sv == nullptr ? 0 : number(*sv)) != 1 ||
        (sq == nullptr ? 0 : number(*sq)) != input_sequence) {
        throw std::invalid_argument("invalid or non-contiguous event sequence");
    }
    const std::uint64_t bytes = number(e.at("bytes"));
    const json_min::value* pb = e.find("page_bytes");
    const std::uint64_t page = pb == nullptr ? bytes : number(*pb);
    const json_min::value* op = e.find("operation");
    std::string operation;
    if (op != nullptr) {
        if (op->kind != json_min::value::string_t) {
            throw std::runtime_error("type_error: operation is not a string");
        }
        operation = op->s;
    }
    if (bytes == 0 || page == 0 || page > std::numeric_limits<std::uint32_t>::max() ||
        bytes % page != 0 || page % 512 != 0 || (operation != "read" && operation != "write")) {
        throw std::invalid_argument("invalid event/page size or operation");
    }
    const std::uint64_t address = number(e.at("logical_address"));
    if (address % page != 0 || bytes > std::numeric_limits<std::uint64_t>::max() - address) {
        throw std::invalid_argument("event range is invalid or misaligned");
    }
    return {address, bytes, static_cast<std::uint32_t>(page), operation == "write"};
}

using cli_json::quote;
using cli_json::real;

// HybridSampler(warmup, rate, 0).reference(sequence - 1, access) for every
// page request in order (hbf_trace_timing.cpp:154-155, 181-206), on the GPU.
std::vector<std::uint8_t> sample_requests(const hbfamd::profile& prof, const std::vector<event>& evs)
{
    std::vector<hbfsim_amd_access_class> access;
    for (const event& ev : evs) {
        const hbfsim_amd_access_class a{ev.write ? 1u : 0u,
                                        static_cast<std::uint32_t>(ev.page_bytes), 0u, 0u};
        access.insert(access.end(), ev.bytes / ev.page_bytes, a);
    }
    std::vector<std::uint8_t> flags(access.size(), 0);
    if (access.empty()) {
        return flags;
    }
    if (access.size() >= (std::size_t{1} << 32)) {
        throw std::runtime_error("hybrid mode takes fewer than 2^32 page requests");
    }
    hbfsim_amd_sampler* sampler = nullptr;
    if (hbfsim_amd_sampler_create(prof.reference_warmup_requests, prof.reference_sample_rate, 0,
                                  &sampler) != HBFSIM_OK) {
        throw std::invalid_argument("sample_rate must be in [0, 1]");
    }
    hbfsim_amd_access_class* d_access = nullptr;
    std::uint8_t* d_flags = nullptr;
    hipError_t err = hipMalloc(reinterpret_cast<void**>(&d_access), access.size() * sizeof(access[0]));
    if (err == hipSuccess) err = hipMalloc(reinterpret_cast<void**>(&d_flags), flags.size());
    if (err == hipSuccess)
        err = hipMemcpy(d_access, access.data(), access.size() * sizeof(access[0]),
                        hipMemcpyHostToDevice);
    int st = err == hipSuccess ? HBFSIM_OK : HBFSIM_CUDA_ERROR;
    if (st == HBFSIM_OK) {
        st = hbfsim_amd_sampler_reference(sampler, d_access, nullptr, 0, access.size(), d_flags,
                                          nullptr, nullptr);
    }
    if (st == HBFSIM_OK && hipMemcpy(flags.data(), d_flags, flags.size(), hipMemcpyDeviceToHost) !=
                               hipSuccess) {
        st = HBFSIM_CUDA_ERROR;
    }
    (void)hipFree(d_access);
    (void)hipFree(d_flags);
    hbfsim_amd_sampler_destroy(sampler);
    if (st != HBFSIM_OK) {
        throw std::runtime_error("the GPU sampler failed (hybrid mode needs a GPU)");
    }
    return flags;
}

}  // namespace

// The library's engine as the detailed model of hybrid mode: one range over
// the profile's capacity, so a request's media page is its logical address
// divided by the page size; each picked page request is one record.
class detailed_engine {
public:
    detailed_engine(const options& o, const hbfamd::profile& prof)
    {
        const std::string dir = std::filesystem::temp_directory_path().string();
        const hbfsim_options co{o.profile_path.c_str(), dir.c_str(), HBFSIM_MODEL_FAST, 64,
                                1000000000ull};
        if (hbfsim_context_create(&co, &ctx_) != HBFSIM_OK) {
            throw std::runtime_error("the detailed engine failed to start (it needs a GPU)");
        }
        const hbfsim_range_options ro{HBFSIM_RANGE_MODE_TIMING, HBFSIM_RANGE_READ_WRITE,
                                      HBFSIM_CACHE_POLICY_NONE, 0};
        if (hbfsim_register_device(ctx_, reinterpret_cast<void*>(kBase), prof.capacity_bytes,
                                   &ro) != HBFSIM_OK) {
            hbfsim_context_destroy(ctx_);
            throw std::runtime_error("the detailed engine refused the profile's capacity");
        }
    }
    ~detailed_engine() { hbfsim_context_destroy(ctx_); }
    detailed_engine(const detailed_engine&) = delete;
    detailed_engine& operator=(const detailed_engine&) = delete;

    // Completion (ns, rounded up) of one page request arriving at arrival_ns.
    std::uint64_t complete(std::uint64_t logical, std::uint32_t page_bytes, bool write,
                           std::uint64_t arrival_ns)
    {
        if (arrival_ns > std::numeric_limits<std::uint64_t>::max() / 1000) {
            throw std::overflow_error("demand clock beyond the engine's picosecond range");
        }
        const hbf_record32 r{kBase + logical, page_bytes, arrival_ns * 1000u, write ? 1u : 0u};
        std::uint64_t done_ps = 0;
        std::uint8_t status = 0;
        if (hbfsim_amd_run(ctx_, &r, 1, &done_ps, &status, 0, nullptr) != HBFSIM_OK ||
            (status & 3u) != HBFSIM_AMD_MODELED) {
            throw std::runtime_error("the detailed engine did not time a page request");
        }
        return done_ps / 1000 + (done_ps % 1000 != 0 ? 1u : 0u);
    }

private:
    static constexpr std::uint64_t kBase = 0x4000'0000'0000ull;
    hbfsim_context* ctx_ = nullptr;
};

int main(int argc, char** argv)
{
    try {
        const options o = parse_options(argc, argv);
        const hbfamd::profile prof = hbfamd::load_profile(o.profile_path);
        std::ifstream in(o.events_path);
        if (!in) {
            throw std::runtime_error("failed to open timing event JSONL");
        }
        if (o.mode == "mqsim") {
            throw std::runtime_error("MQSim reference timing is not part of this engine");
        }
        std::uint64_t input_events = 0, sequence = 0, clock_ns = 0, service_ns = 0;
        std::uint64_t fast_requests = 0, reference_requests = 0;
        std::vector<event> evs;  // hybrid mode: the sampler takes every request at once
        std::string line;
        const auto t0 = std::chrono::steady_clock::now();
        // the fast model of one event's pages (hbf_trace_timing.cpp:214-231)
        const auto fast = [&](const event& ev, std::uint64_t pages) {
            const std::uint64_t base = ev.write ? prof.program_latency_ns : prof.read_latency_ns;
            const std::uint64_t service =
                fast_service(base, ev.page_bytes, prof.aggregate_bandwidth_bytes_per_s);
            const std::uint64_t t = transfer_ns(ev.page_bytes, prof.aggregate_bandwidth_bytes_per_s);
            const std::uint64_t exposed = base > t ? base : t;
            if (service == 0 || exposed == 0) {
                throw std::runtime_error("fast model rejected an event");
            }
            service_ns = sat_add_n(service_ns, pages, service);
            clock_ns = sat_add_n(clock_ns, pages, exposed);
            fast_requests += pages;
        };
        while (std::getline(in, line)) {
            if (line.empty()) {
                continue;
            }
            ++input_events;
            const event ev = parse_event(json_min::parse(line), input_events);
            if (ev.page_bytes != prof.page_bytes || ev.logical_address + ev.bytes > prof.capacity_bytes) {
                throw std::invalid_argument(
                    "event page size or range differs from the frozen profile");
            }
            const std::uint64_t pages = ev.bytes / ev.page_bytes;
            sequence += pages;
            if (o.mode == "hybrid") {
                evs.push_back(ev);
            } else {
                fast(ev, pages);
            }
        }
        if (o.mode == "hybrid") {
            const std::vector<std::uint8_t> sampled = sample_requests(prof, evs);
            detailed_engine detail(o, prof);
            std::size_t k = 0;
            for (const event& ev : evs) {
                const std::uint64_t pages = ev.bytes / ev.page_bytes;
                std::uint64_t run = 0;  // pending fast pages, in order
                for (std::uint64_t p = 0; p < pages; ++p, ++k) {
                    if (!sampled[k]) {
                        ++run;
                        continue;
                    }
                    fast(ev, run);
                    run = 0;
                    // hbf_trace_timing.cpp:203-208: the detailed engine's
                    // completion becomes the demand clock
                    const std::uint64_t arrival = clock_ns;
                    const std::uint64_t done =
                        detail.complete(ev.logical_address + p * ev.page_bytes, ev.page_bytes,
                                        ev.write, arrival);
                    clock_ns = done;
                    service_ns = sat_add_n(service_ns, 1, done - arrival);
                    ++reference_requests;
                }
                fast(ev, run);
            }
        }
        const auto wall = static_cast<std::uint64_t>(
            std::chrono::duration_cast<std::chrono::nanoseconds>(
                std::chrono::steady_clock::now() - t0)
                .count());
        std::ostringstream os;
        os << "{\n"
           << "  \"demand_exposed_stall_ns\": " << clock_ns << ",\n"
           << "  \"emulator_dispatcher_wall_time_ns\": " << wall << ",\n"
           << "  \"engine\": \"" << (o.mode == "hybrid" ? "hbf-hybrid" : "hbf-fast") << "\",\n"
           << "  \"modeled_device_service_ns\": " << service_ns << ",\n"
           << "  \"profile\": " << quote(prof.name) << ",\n"
           << "  \"reference_sample_rate\": " << real(prof.reference_sample_rate) << ",\n"
           << (o.mode == "hybrid"
                   ? "  \"reference_timing\": \"hbf-amd-engine (per-plane tR/tPROG, page "
                     "register and channel cursor on the GPU, in place of MQSim)\",\n"
                   : "")
           << "  \"reference_warmup_requests\": " << prof.reference_warmup_requests << ",\n"
           << "  \"requests\": {\n"
           << "    \"fast\": " << fast_requests << ",\n"
           << "    \"input_expert_misses\": " << input_events << ",\n"
           << "    \"reference\": " << reference_requests << ",\n"
           << "    \"submitted\": " << sequence << "\n"
           << "  },\n"
           << "  \"scheduling_semantics\": \"ordered blocking demand misses with no compute "
              "gaps\",\n"
           << "  \"schema_version\": 1,\n"
           << "  \"status\": \"PASS\"\n"
           << "}\n";
        std::cout << os.str();
        return 0;
    } catch (const std::invalid_argument& e) {
        std::cerr << "hbf_trace_timing: " << e.what() << '\n';
        return 64;
    } catch (const std::exception& e) {
        std::cerr << "hbf_trace_timing: " << e.what() << '\n';
        return 2;
    }
}
