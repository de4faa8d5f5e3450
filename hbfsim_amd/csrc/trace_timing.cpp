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
// is host code.  hybrid and mqsim modes need the MQSim reference (hybrid
// sends the first request of every access class to it,
// calibrator.cpp:83-96), which is not part of this build: they exit 2.
//
// Output: the reference's JSON report, keys sorted and two-space indented as
// nlohmann::json::dump(2) prints it.  Exit 64 on invalid arguments or
// events (std::invalid_argument in the reference), 2 on other errors.
#include "json_min.hpp"
#include "profile.hpp"

#include <charconv>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <fstream>
#include <iostream>
#include <limits>
#include <sstream>
#include <stdexcept>
#include <string>
#include <string_view>

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

std::string quote(const std::string& s)
{
    std::string out = "\"";
    for (const char ch : s) {
        const auto c = static_cast<unsigned char>(ch);
        switch (c) {
        case '"': out += "\\\""; break;
        case '\\': out += "\\\\"; break;
        case '\b': out += "\\b"; break;
        case '\f': out += "\\f"; break;
        case '\n': out += "\\n"; break;
        case '\r': out += "\\r"; break;
        case '\t': out += "\\t"; break;
        default:
            if (c < 0x20) {
                char buf[8];
                std::snprintf(buf, sizeof buf, "\\u%04x", c);
                out += buf;
            } else {
                out += ch;
            }
        }
    }
    return out + "\"";
}

// A double as nlohmann::json prints it: the shortest round-trip form, with
// ".0" appended when that reads as an integer.
std::string real(double v)
{
    char buf[64];
    const auto r = std::to_chars(buf, buf + sizeof buf, v);
    std::string s(buf, r.ptr);
    if (s.find_first_of(".eEn") == std::string::npos) {
        s += ".0";
    }
    return s;
}

}  // namespace

int main(int argc, char** argv)
{
    try {
        const options o = parse_options(argc, argv);
        const hbfamd::profile prof = hbfamd::load_profile(o.profile_path);
        std::ifstream in(o.events_path);
        if (!in) {
            throw std::runtime_error("failed to open timing event JSONL");
        }
        if (o.mode != "fast") {
            throw std::runtime_error(
                "MQSim reference timing is not part of this engine (mode " + o.mode + ")");
        }
        std::uint64_t input_events = 0, sequence = 0, clock_ns = 0, service_ns = 0;
        std::uint64_t fast_requests = 0;
        std::string line;
        const auto t0 = std::chrono::steady_clock::now();
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
            sequence += pages;
            fast_requests += pages;
        }
        const auto wall = static_cast<std::uint64_t>(
            std::chrono::duration_cast<std::chrono::nanoseconds>(
                std::chrono::steady_clock::now() - t0)
                .count());
        std::ostringstream os;
        os << "{\n"
           << "  \"demand_exposed_stall_ns\": " << clock_ns << ",\n"
           << "  \"emulator_dispatcher_wall_time_ns\": " << wall << ",\n"
           << "  \"engine\": \"hbf-fast\",\n"
           << "  \"modeled_device_service_ns\": " << service_ns << ",\n"
           << "  \"profile\": " << quote(prof.name) << ",\n"
           << "  \"reference_sample_rate\": " << real(prof.reference_sample_rate) << ",\n"
           << "  \"reference_warmup_requests\": " << prof.reference_warmup_requests << ",\n"
           << "  \"requests\": {\n"
           << "    \"fast\": " << fast_requests << ",\n"
           << "    \"input_expert_misses\": " << input_events << ",\n"
           << "    \"reference\": 0,\n"
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
