// api.cpp -- the exported C ABI: the reference's public API and vLLM
// extension, plus the batch timing engine's entry points.
//
// Behaviour follows the reference's context and registry
// (src/cuda_runtime/context.cpp:424-433, 863-1000, 1658-1760, 1909-2110;
// src/cuda_runtime/range_table.cpp:17-198; adapters/vllm/hbfsim_extension.cpp:
// 13-101): out-pointers are nulled before validation, no exception crosses
// the ABI, and errors map to the same hbfsim_error codes.  Creating a context
// and registering ranges need no GPU; the engine and its device memory are
// created on first use.
#include "engine.hpp"
#include "link.hpp"
#include "thermal.hpp"
#include "profile.hpp"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <limits>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#define HBF_API extern "C" __attribute__((visibility("default")))

struct hbfsim_context {
    std::mutex mu;
    hbfamd::profile prof;
    std::string profile_path;
    std::string report_dir;
    std::uint32_t mode{HBFSIM_MODEL_FAST};
    hbfsim_amd_engine_options opts{};
    // registry (range_table.cpp)
    std::vector<hbfamd::range_rec> ranges;  // sorted by base
    std::uint64_t next_file_offset{0};
    std::uint32_t next_range_id{1};
    // engine and accounting
    hbfamd::engine* eng{nullptr};
    hbfsim_amd_report total{};
    hbfsim_stats stats{};
};

struct hbfsim_vllm_session {
    hbfsim_context* context{nullptr};
};

namespace {

constexpr std::uint32_t kRangeCapacity = 32768;  // hbf_device.cuh:21

std::uint64_t gcd64(std::uint64_t a, std::uint64_t b)
{
    while (b != 0) {
        const std::uint64_t t = a % b;
        a = b;
        b = t;
    }
    return a;
}

// context.cpp:975-981
std::uint64_t sample_threshold(double rate)
{
    if (rate >= 1.0) {
        return std::numeric_limits<std::uint64_t>::max();
    }
    return static_cast<std::uint64_t>(
        rate * static_cast<long double>(std::numeric_limits<std::uint64_t>::max()));
}

std::uint32_t log2_exact(std::uint32_t v)
{
    std::uint32_t b = 0;
    while ((1u << b) < v) {
        ++b;
    }
    return b;
}

void default_options(const hbfsim_context* c, hbfsim_amd_engine_options* o)
{
    std::memset(o, 0, sizeof(*o));
    o->struct_size = sizeof(*o);
    o->model = c->prof.empirical.present ? HBFSIM_AMD_MODEL_EMPIRICAL : HBFSIM_AMD_MODEL_HBF;
    o->page_buffers = 1;
    o->plane_contention = 1;
    o->transfer_page = 0;
    o->program_every_write = 0;
    o->flat_geometry = 0;
    o->ways = 1;
    o->xfer_quantum_ps = 1;
    o->channel_bandwidth_bytes_per_s = 0;
    o->tile_records = 0;  // automatic
}

// Resolves profile + options into the kernels' configuration.
int build_config(const hbfsim_context* c, hbfamd::engine_config* cfg)
{
    const hbfamd::profile& p = c->prof;
    const hbfsim_amd_engine_options& o = c->opts;
    hbfamd::engine_config k;
    k.model = o.model;
    if (o.flat_geometry) {
        k.channels = k.ways = k.dies = k.planes = 1;
    } else {
        k.channels = p.channels;
        k.ways = o.ways == 0 ? 1 : o.ways;
        k.dies = p.dies_per_channel;
        k.planes = p.planes_per_die;
    }
    for (int i = 0; i < 4; ++i) {
        k.order[i] = p.axis_order[i];
    }
    k.page_shift = log2_exact(p.page_bytes);
    k.slots = o.page_buffers;
    k.contention = o.plane_contention ? 1u : 0u;
    k.transfer_page = o.transfer_page ? 1u : 0u;
    k.every_write = o.program_every_write ? 1u : 0u;
    k.hybrid = c->mode == HBFSIM_MODEL_HYBRID ? 1u : 0u;
    k.hybrid_warmup = p.reference_warmup_requests;
    k.hybrid_threshold = sample_threshold(p.reference_sample_rate);
    if (p.read_latency_ns > UINT64_MAX / 1000 || p.program_latency_ns > UINT64_MAX / 1000) {
        return HBFSIM_UNSUPPORTED;
    }
    k.read_ps = p.read_latency_ns * 1000ull;
    k.program_ps = p.program_latency_ns * 1000ull;
    const std::uint64_t q = o.xfer_quantum_ps == 0 ? 1 : o.xfer_quantum_ps;
    // xfer_ps = q * ceil(bytes * num / den), bandwidth per channel in B/s:
    //   explicit:  num = 1e12, den = bw * q
    //   default:   aggregate / channels -> num = 1e12 * C, den = aggregate * q
    unsigned __int128 num = 1000000000000ull, den;
    if (o.channel_bandwidth_bytes_per_s != 0) {
        den = static_cast<unsigned __int128>(o.channel_bandwidth_bytes_per_s) * q;
    } else {
        num *= k.channels;
        den = static_cast<unsigned __int128>(p.aggregate_bandwidth_bytes_per_s) * q;
    }
    if (den == 0) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    // reduce by the gcd (both fit 64 bits after reduction in practice)
    std::uint64_t g = 1;
    if (num <= UINT64_MAX && den <= UINT64_MAX) {
        g = gcd64(static_cast<std::uint64_t>(num), static_cast<std::uint64_t>(den));
    }
    num /= g;
    den /= g;
    if (num > UINT64_MAX || den > UINT64_MAX) {
        return HBFSIM_UNSUPPORTED;
    }
    k.xfer_num = static_cast<std::uint64_t>(num);
    k.xfer_den = static_cast<std::uint64_t>(den);
    k.xfer_quantum = q;
    k.tile = o.tile_records;  // 0: chosen per run from the batch size
    k.grouping = o.warp_grouping;
    // page registers hold page + 1 in 32 bits on the device
    if ((p.capacity_bytes >> k.page_shift) >= 0xffffffffull) {
        return HBFSIM_UNSUPPORTED;
    }
    k.media_pages = p.capacity_bytes >> k.page_shift;
    if (p.empirical.present) {
        for (int i = 0; i < 6; ++i) {
            k.emp_pages[i] = p.empirical.read_curve[i].pages;
            k.emp_cum_ns[i] = p.empirical.read_curve[i].cumulative_ns;
        }
    }
    k.emp_program_ns = p.program_latency_ns;
    *cfg = k;
    return HBFSIM_OK;
}

int ensure_engine(hbfsim_context* c)
{
    if (c->eng != nullptr) {
        return HBFSIM_OK;
    }
    hbfamd::engine_config cfg;
    int st = build_config(c, &cfg);
    if (st != HBFSIM_OK) {
        return st;
    }
    st = hbfamd::engine_create(cfg, &c->eng);
    if (st != HBFSIM_OK) {
        return st;
    }
    return hbfamd::engine_set_ranges(c->eng, c->ranges);
}

void add_report(hbfsim_amd_report& t, const hbfsim_amd_report& r)
{
    t.records += r.records;
    t.modeled += r.modeled;
    t.bypass += r.bypass;
    t.unsupported += r.unsupported;
    t.reads += r.reads;
    t.writes += r.writes;
    t.page_hits += r.page_hits;
    t.programs += r.programs;
    t.hybrid_sampled += r.hybrid_sampled;
    t.makespan_ps = std::max(t.makespan_ps, r.makespan_ps);
    const std::uint64_t lo = t.latency_sum_lo + r.latency_sum_lo;
    t.latency_sum_hi += r.latency_sum_hi + (lo < t.latency_sum_lo ? 1u : 0u);
    t.latency_sum_lo = lo;
    t.latency_max_ps = std::max(t.latency_max_ps, r.latency_max_ps);
    t.service_sum_ps += r.service_sum_ps;
    t.grouped += r.grouped;
}

// hbfsim_stats as the reference fills it (context.cpp:1983-2004): the request
// counters count ring requests, i.e. the requests the hybrid sampler sends to
// the detailed model (hbf_device.cu:782-787 -> resolve_leader), so they stay 0
// in fast mode; fast_requests counts the fast-model resolutions
// (hbf_device.cu:951), one per media request: lanes that joined a warp
// group's request are not resolutions of their own.  A sampled request is
// submitted and completed in the same run here.
void account(hbfsim_context* c, const hbfsim_amd_report& r)
{
    add_report(c->total, r);
    c->stats.requests_submitted += r.hybrid_sampled;
    c->stats.requests_completed += r.hybrid_sampled;
    c->stats.fast_requests += r.modeled - r.grouped - r.hybrid_sampled;
    c->stats.reference_requests += r.hybrid_sampled;
    c->stats.fast_modeled_ns += r.service_sum_ps / 1000u;
}

void write_report(const hbfsim_context* c)
{
    std::error_code ec;
    const std::filesystem::path path =
        std::filesystem::path(c->report_dir) / "hbfsim-amd-report.json";
    std::ofstream out(path);
    if (!out) {
        return;
    }
    const hbfsim_amd_report& t = c->total;
    out << "{\"schema_version\":1,\"engine\":\"hbfsim-amd\",\"profile\":\"" << c->prof.name
        << "\",\"records\":" << t.records << ",\"modeled\":" << t.modeled
        << ",\"bypass\":" << t.bypass << ",\"unsupported\":" << t.unsupported
        << ",\"reads\":" << t.reads << ",\"writes\":" << t.writes
        << ",\"page_hits\":" << t.page_hits << ",\"programs\":" << t.programs
        << ",\"hybrid_sampled\":" << t.hybrid_sampled << ",\"makespan_ps\":" << t.makespan_ps
        << ",\"latency_sum_lo\":" << t.latency_sum_lo
        << ",\"latency_sum_hi\":" << t.latency_sum_hi
        << ",\"latency_max_ps\":" << t.latency_max_ps
        << ",\"service_sum_ps\":" << t.service_sum_ps << ",\"grouped\":" << t.grouped
        << "}\n";
}

}  // namespace

// ---- 1. reference API -------------------------------------------------

HBF_API uint32_t hbfsim_abi_version(void) { return 1u; }

HBF_API int hbfsim_context_create(const hbfsim_options* options, hbfsim_context** out)
{
    if (out != nullptr) {
        *out = nullptr;
    }
    // context.cpp:424-433
    if (out == nullptr || options == nullptr || options->profile_path == nullptr ||
        options->profile_path[0] == '\0' || options->report_dir == nullptr ||
        options->report_dir[0] == '\0' || options->mode > HBFSIM_MODEL_HYBRID ||
        options->ring_capacity < 2 || options->ring_capacity > 4096 ||
        (options->ring_capacity & (options->ring_capacity - 1)) != 0 ||
        options->request_timeout_ns == 0) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    try {
        auto* c = new (std::nothrow) hbfsim_context;
        if (c == nullptr) {
            return HBFSIM_IO_ERROR;
        }
        try {
            c->prof = hbfamd::load_profile(options->profile_path);
        } catch (const hbfamd::profile_error&) {
            delete c;
            return HBFSIM_INVALID_ARGUMENT;
        }
        if (options->mode == HBFSIM_MODEL_REFERENCE) {
            // The reference mode runs MQSim in a daemon; MQSim is not part
            // of this engine.
            delete c;
            return HBFSIM_UNSUPPORTED;
        }
        std::error_code ec;
        std::filesystem::create_directories(options->report_dir, ec);
        if (ec) {
            delete c;
            return HBFSIM_IO_ERROR;
        }
        c->profile_path = options->profile_path;
        c->report_dir = options->report_dir;
        c->mode = options->mode;
        default_options(c, &c->opts);
        *out = c;
        return HBFSIM_OK;
    } catch (...) {
        return HBFSIM_IO_ERROR;
    }
}

HBF_API int hbfsim_register_device(hbfsim_context* c, void* device_ptr, size_t length,
                                   const hbfsim_range_options* options)
{
    // context.cpp:1658-1670
    if (c == nullptr || device_ptr == nullptr || length == 0 || options == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    if (options->mode != HBFSIM_RANGE_MODE_TIMING) {
        return options->mode == HBFSIM_RANGE_MODE_CAPACITY ? HBFSIM_UNSUPPORTED
                                                           : HBFSIM_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(c->mu);
    // range_table.cpp:17-118
    const std::uint64_t base = reinterpret_cast<std::uintptr_t>(device_ptr);
    const std::uint64_t page = c->prof.page_bytes;
    if (page == 0 || length > UINT64_MAX - base || options->permissions == 0 ||
        (options->permissions & ~static_cast<std::uint32_t>(HBFSIM_RANGE_READ_WRITE)) != 0 ||
        options->cache_policy != HBFSIM_CACHE_POLICY_NONE) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    if (c->ranges.size() == kRangeCapacity) {
        return HBFSIM_UNSUPPORTED;
    }
    const std::uint64_t len = length;
    if (len > UINT64_MAX - (page - 1)) {
        return HBFSIM_UNSUPPORTED;
    }
    const std::uint64_t extent = ((len + page - 1) / page) * page;
    if (c->next_file_offset > c->prof.capacity_bytes ||
        extent > c->prof.capacity_bytes - c->next_file_offset) {
        return HBFSIM_UNSUPPORTED;
    }
    std::size_t index = 0;
    {
        std::size_t lo = 0, hi = c->ranges.size();
        while (lo < hi) {
            const std::size_t mid = (lo + hi) / 2;
            if (c->ranges[mid].base < base) {
                lo = mid + 1;
            } else {
                hi = mid;
            }
        }
        index = lo;
    }
    const std::uint64_t end = base + len;
    if ((index != 0 && c->ranges[index - 1].base + c->ranges[index - 1].length > base) ||
        (index != c->ranges.size() && end > c->ranges[index].base)) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    hbfamd::range_rec r{};
    r.base = base;
    r.length = len;
    r.file_offset = c->next_file_offset;
    r.range_id = c->next_range_id;
    r.mode = options->mode;
    r.permissions = options->permissions;
    r.cache_policy = options->cache_policy;
    r.stream_id = options->stream_id;
    r.flags = 0;
    r.page_bytes = page;
    try {
        c->ranges.insert(c->ranges.begin() + static_cast<std::ptrdiff_t>(index), r);
    } catch (...) {
        return HBFSIM_IO_ERROR;
    }
    c->next_range_id += 1;
    c->next_file_offset += extent;
    if (c->eng != nullptr) {
        hbfamd::engine_set_ranges(c->eng, c->ranges);
    }
    return HBFSIM_OK;
}

HBF_API int hbfsim_map_file(hbfsim_context* c, const char* path, uint64_t file_offset,
                            size_t length, const hbfsim_range_options* options,
                            void** logical_device_ptr_out)
{
    // context.cpp:1719-1745
    if (logical_device_ptr_out != nullptr) {
        *logical_device_ptr_out = nullptr;
    }
    if (c == nullptr || path == nullptr || path[0] == '\0' || length == 0 || options == nullptr ||
        logical_device_ptr_out == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    if (options->mode != HBFSIM_RANGE_MODE_CAPACITY) {
        return options->mode == HBFSIM_RANGE_MODE_TIMING ? HBFSIM_UNSUPPORTED
                                                         : HBFSIM_INVALID_ARGUMENT;
    }
    if ((options->permissions != HBFSIM_RANGE_READ &&
         options->permissions != HBFSIM_RANGE_READ_WRITE) ||
        options->cache_policy != HBFSIM_CACHE_POLICY_NONE ||
        file_offset > UINT64_MAX - length) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    return HBFSIM_UNSUPPORTED;
}

HBF_API int hbfsim_flush(hbfsim_context* c)
{
    if (c == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(c->mu);
    if (c->eng != nullptr) {
        const int st = hbfamd::engine_synchronize(c->eng);
        if (st != HBFSIM_OK) {
            return st;
        }
    }
    write_report(c);
    return HBFSIM_OK;
}

HBF_API int hbfsim_get_stats(hbfsim_context* c, hbfsim_stats* out)
{
    if (c == nullptr || out == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(c->mu);
    *out = c->stats;
    return HBFSIM_OK;
}

HBF_API int hbfsim_get_capacity_stats_v1(hbfsim_context* c, hbfsim_capacity_stats_v1* out)
{
    if (c == nullptr || out == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    std::memset(out, 0, sizeof(*out));
    out->struct_size = sizeof(*out);
    out->version = HBFSIM_CAPACITY_STATS_V1_VERSION;
    out->enabled = 0;
    out->page_bytes = c->prof.page_bytes;
    return HBFSIM_OK;
}

HBF_API int hbfsim_unregister(hbfsim_context* c, void* range_base)
{
    if (c == nullptr || range_base == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(c->mu);
    const std::uint64_t base = reinterpret_cast<std::uintptr_t>(range_base);
    for (std::size_t i = 0; i < c->ranges.size(); ++i) {
        if (c->ranges[i].base == base) {
            c->ranges.erase(c->ranges.begin() + static_cast<std::ptrdiff_t>(i));
            if (c->eng != nullptr) {
                hbfamd::engine_set_ranges(c->eng, c->ranges);
            }
            return HBFSIM_OK;
        }
    }
    return HBFSIM_INVALID_ARGUMENT;
}

HBF_API void hbfsim_context_destroy(hbfsim_context* c)
{
    if (c == nullptr) {
        return;
    }
    if (c->total.records != 0) {
        write_report(c);
    }
    hbfamd::engine_destroy(c->eng);
    delete c;
}

// ---- 2. vLLM extension ------------------------------------------------

HBF_API uint32_t hbfsim_vllm_abi_version(void) { return 2u; }

HBF_API int hbfsim_vllm_session_create(const hbfsim_vllm_options* options,
                                       hbfsim_vllm_session** out)
{
    if (out == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    *out = nullptr;
    if (options == nullptr || options->profile_path == nullptr ||
        options->profile_path[0] == '\0' || options->report_dir == nullptr ||
        options->report_dir[0] == '\0' || options->ring_capacity == 0 ||
        options->timing_model > HBFSIM_MODEL_HYBRID || options->request_timeout_ns == 0) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    auto* session = new (std::nothrow) hbfsim_vllm_session;
    if (session == nullptr) {
        return HBFSIM_IO_ERROR;
    }
    const hbfsim_options copt{options->profile_path, options->report_dir, options->timing_model,
                              options->ring_capacity, options->request_timeout_ns};
    const int st = hbfsim_context_create(&copt, &session->context);
    if (st != HBFSIM_OK) {
        delete session;
        return st;
    }
    *out = session;
    return HBFSIM_OK;
}

HBF_API int hbfsim_vllm_register_storage(hbfsim_vllm_session* session, uintptr_t device_address,
                                         size_t bytes)
{
    if (session == nullptr || session->context == nullptr || device_address == 0 || bytes == 0) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    const hbfsim_range_options o{HBFSIM_RANGE_MODE_TIMING, HBFSIM_RANGE_READ,
                                 HBFSIM_CACHE_POLICY_NONE, 0};
    return hbfsim_register_device(session->context, reinterpret_cast<void*>(device_address), bytes,
                                  &o);
}

HBF_API int hbfsim_vllm_session_close(hbfsim_vllm_session** session)
{
    if (session == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    if (*session == nullptr) {
        return HBFSIM_OK;
    }
    hbfsim_context_destroy((*session)->context);
    (*session)->context = nullptr;
    delete *session;
    *session = nullptr;
    return HBFSIM_OK;
}

HBF_API const char* hbfsim_vllm_status_string(int status)
{
    switch (status) {
    case HBFSIM_OK: return "ok";
    case HBFSIM_INVALID_ARGUMENT: return "invalid_argument";
    case HBFSIM_IO_ERROR: return "io_error";
    case HBFSIM_CUDA_ERROR: return "cuda_error";
    case HBFSIM_TIMEOUT: return "timeout";
    case HBFSIM_UNSUPPORTED: return "unsupported";
    case HBFSIM_DAEMON_LOST: return "daemon_lost";
    default: return "unknown";
    }
}

HBF_API hbfsim_context* hbfsim_vllm_session_context(hbfsim_vllm_session* session)
{
    return session == nullptr ? nullptr : session->context;
}

// ---- 3. batch engine --------------------------------------------------

HBF_API int hbfsim_amd_default_engine_options(const hbfsim_context* c,
                                              hbfsim_amd_engine_options* out)
{
    if (c == nullptr || out == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    default_options(c, out);
    return HBFSIM_OK;
}

HBF_API int hbfsim_amd_set_engine_options(hbfsim_context* c,
                                          const hbfsim_amd_engine_options* o)
{
    if (c == nullptr || o == nullptr || o->struct_size != sizeof(hbfsim_amd_engine_options)) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    if (o->model > HBFSIM_AMD_MODEL_EMPIRICAL || o->page_buffers > 2 ||
        (o->tile_records % 64) != 0 || o->warp_grouping > 1) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    if (o->model == HBFSIM_AMD_MODEL_EMPIRICAL && !c->prof.empirical.present) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(c->mu);
    hbfsim_amd_engine_options saved = c->opts;
    c->opts = *o;
    hbfamd::engine_config cfg;
    const int st = build_config(c, &cfg);
    if (st != HBFSIM_OK) {
        c->opts = saved;
        return st;
    }
    hbfamd::engine_destroy(c->eng);
    c->eng = nullptr;
    std::memset(&c->total, 0, sizeof(c->total));
    return HBFSIM_OK;
}

HBF_API int hbfsim_amd_get_engine_options(const hbfsim_context* c,
                                          hbfsim_amd_engine_options* out)
{
    if (c == nullptr || out == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    *out = c->opts;
    return HBFSIM_OK;
}

HBF_API int hbfsim_amd_run_device(hbfsim_context* c, const hbf_record32* records, size_t n,
                                  uint64_t* completion_ps, uint8_t* status, uint64_t base_ps,
                                  void* stream, hbfsim_amd_report* report)
{
    if (report != nullptr) {
        std::memset(report, 0, sizeof(*report));
    }
    if (c == nullptr || (n != 0 && (records == nullptr || completion_ps == nullptr))) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(c->mu);
    int st = ensure_engine(c);
    if (st != HBFSIM_OK) {
        return st;
    }
    hbfsim_amd_report r{};
    st = hbfamd::engine_run(c->eng, records, n, completion_ps, status, base_ps, stream, &r);
    if (st != HBFSIM_OK) {
        return st;
    }
    account(c, r);
    if (report != nullptr) {
        *report = r;
    }
    return HBFSIM_OK;
}

HBF_API int hbfsim_amd_run_device_packed(hbfsim_context* c, const hbf_record16* records,
                                         size_t n, uint64_t* completion_ps, uint8_t* status,
                                         uint64_t base_ps, void* stream,
                                         hbfsim_amd_report* report)
{
    if (report != nullptr) {
        std::memset(report, 0, sizeof(*report));
    }
    if (c == nullptr || (n != 0 && (records == nullptr || completion_ps == nullptr))) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(c->mu);
    int st = ensure_engine(c);
    if (st != HBFSIM_OK) {
        return st;
    }
    hbfsim_amd_report r{};
    st = hbfamd::engine_run_packed(c->eng, records, n, completion_ps, status, base_ps, stream,
                                   &r);
    if (st != HBFSIM_OK) {
        return st;
    }
    account(c, r);
    if (report != nullptr) {
        *report = r;
    }
    return HBFSIM_OK;
}

HBF_API int hbfsim_amd_run_device_packed_noalloc(hbfsim_context* c, const hbf_record16* records,
                                                 size_t n, uint64_t* completion_ps,
                                                 uint8_t* status, uint64_t base_ps, void* stream,
                                                 hbfsim_amd_report* report)
{
    // a refused call leaves the caller's report, like the context, untouched
    if (c == nullptr || (n != 0 && (records == nullptr || completion_ps == nullptr))) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(c->mu);
    if (c->eng == nullptr) {
        return HBFSIM_UNSUPPORTED;  // creating the engine allocates
    }
    hbfsim_amd_report r{};
    const int st = hbfamd::engine_run_packed_noalloc(c->eng, records, n, completion_ps, status,
                                                     base_ps, stream, &r);
    if (st != HBFSIM_OK) {
        return st;
    }
    account(c, r);
    if (report != nullptr) {
        *report = r;
    }
    return HBFSIM_OK;
}

HBF_API int hbfsim_amd_run(hbfsim_context* c, const hbf_record32* records, size_t n,
                           uint64_t* completion_ps, uint8_t* status, uint64_t base_ps,
                           hbfsim_amd_report* report)
{
    if (report != nullptr) {
        std::memset(report, 0, sizeof(*report));
    }
    if (c == nullptr || (n != 0 && (records == nullptr || completion_ps == nullptr))) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(c->mu);
    int st = ensure_engine(c);
    if (st != HBFSIM_OK) {
        return st;
    }
    hbfsim_amd_report r{};
    st = hbfamd::engine_run_host(c->eng, records, n, completion_ps, status, base_ps, &r);
    if (st != HBFSIM_OK) {
        return st;
    }
    account(c, r);
    if (report != nullptr) {
        *report = r;
    }
    return HBFSIM_OK;
}

// ---- EQ3 thermal grid and the thermal-coupled run ----------------------

struct hbfsim_amd_thermal {
    hbfamd::thermal* impl;
};

HBF_API int hbfsim_amd_thermal_create(const hbfsim_amd_thermal_grid* grid,
                                      hbfsim_amd_thermal** out)
{
    if (out != nullptr) {
        *out = nullptr;
    }
    if (grid == nullptr || out == nullptr || grid->struct_size != sizeof(*grid)) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    try {
        hbfamd::thermal* impl = nullptr;
        const int st = hbfamd::thermal_create(*grid, &impl);
        if (st != HBFSIM_OK) {
            return st;
        }
        *out = new hbfsim_amd_thermal{impl};
        return HBFSIM_OK;
    } catch (...) {
        return HBFSIM_IO_ERROR;
    }
}

HBF_API int hbfsim_amd_thermal_step(hbfsim_amd_thermal* t, const double* d_power,
                                    double* d_temperature, uint64_t steps, void* stream)
{
    if (t == nullptr || d_power == nullptr || d_temperature == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    return hbfamd::thermal_step(t->impl, d_power, d_temperature, steps, stream);
}

HBF_API int hbfsim_amd_thermal_last_ms(const hbfsim_amd_thermal* t, float* ms)
{
    if (t == nullptr || ms == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    *ms = hbfamd::thermal_last_step_ms(t->impl);
    return HBFSIM_OK;
}

HBF_API int hbfsim_amd_thermal_last_launches(const hbfsim_amd_thermal* t, uint64_t* launches)
{
    if (t == nullptr || launches == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    *launches = hbfamd::thermal_last_launches(t->impl);
    return HBFSIM_OK;
}

HBF_API void hbfsim_amd_thermal_destroy(hbfsim_amd_thermal* t)
{
    if (t == nullptr) {
        return;
    }
    hbfamd::thermal_destroy(t->impl);
    delete t;
}

HBF_API int hbfsim_amd_run_coupled(hbfsim_context* c, hbfsim_amd_thermal* t,
                                   const hbfsim_amd_reliability_options* o,
                                   const hbf_record32* records, size_t n,
                                   uint64_t* completion_ps, double* d_temperature,
                                   uint64_t* age_ps, void* stream,
                                   hbfsim_amd_coupled_report* report,
                                   hbfsim_amd_report* engine_report)
{
    if (report != nullptr) {
        std::memset(report, 0, sizeof(*report));
    }
    if (engine_report != nullptr) {
        std::memset(engine_report, 0, sizeof(*engine_report));
    }
    if (c == nullptr || t == nullptr || o == nullptr || o->struct_size != sizeof(*o)) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(c->mu);
    int st = ensure_engine(c);
    if (st != HBFSIM_OK) {
        return st;
    }
    try {
        hbfsim_amd_report r{};
        st = hbfamd::coupled_run(c->eng, hbfamd::engine_get_config(c->eng), t->impl, *o, records,
                                 n, completion_ps, d_temperature, age_ps, stream, report, &r);
        if (st != HBFSIM_OK) {
            return st;
        }
        account(c, r);
        if (engine_report != nullptr) {
            *engine_report = r;
        }
        return HBFSIM_OK;
    } catch (...) {
        return HBFSIM_IO_ERROR;
    }
}

HBF_API int hbfsim_amd_coupled_last_ms(const hbfsim_amd_thermal* t, float* ms, int max_phases)
{
    if (t == nullptr || ms == nullptr || max_phases < 0) {
        return -1;
    }
    return hbfamd::coupled_last_ms(t->impl, ms, max_phases);
}

HBF_API int hbfsim_amd_coupled_trace(const hbfsim_amd_thermal* t, double* hot, size_t hot_count,
                                     uint8_t* level, size_t level_count, uint8_t* refresh,
                                     size_t refresh_count, uint64_t* windows, uint32_t* dies)
{
    if (t == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    return hbfamd::coupled_trace(t->impl, hot, hot_count, level, level_count, refresh,
                                 refresh_count, windows, dies);
}

HBF_API int hbfsim_amd_get_report(const hbfsim_context* c, hbfsim_amd_report* out)
{
    if (c == nullptr || out == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    *out = c->total;
    return HBFSIM_OK;
}

HBF_API int hbfsim_amd_get_geometry(const hbfsim_context* c, uint32_t* channels,
                                    uint32_t* planes)
{
    if (c == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    hbfamd::engine_config cfg;
    const int st = build_config(c, &cfg);
    if (st != HBFSIM_OK) {
        return st;
    }
    if (channels != nullptr) *channels = cfg.n_channels();
    if (planes != nullptr) *planes = cfg.n_planes();
    return HBFSIM_OK;
}

HBF_API int hbfsim_amd_get_busy_totals(hbfsim_context* c, uint64_t* plane_ps, size_t planes,
                                       uint64_t* channel_ps, size_t channels)
{
    if (c == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(c->mu);
    const int st = ensure_engine(c);
    if (st != HBFSIM_OK) {
        return st;
    }
    return hbfamd::engine_get_busy_totals(c->eng, plane_ps, planes, channel_ps, channels);
}

HBF_API int hbfsim_amd_get_state(hbfsim_context* c, uint64_t* plane_busy, uint64_t* plane_tags,
                                 uint64_t* channel_cursor, uint64_t* sequence,
                                 uint64_t* burst_state)
{
    if (c == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(c->mu);
    const int st = ensure_engine(c);
    if (st != HBFSIM_OK) {
        return st;
    }
    return hbfamd::engine_get_state(c->eng, plane_busy, plane_tags, channel_cursor, sequence,
                                    burst_state);
}

HBF_API int hbfsim_amd_set_state(hbfsim_context* c, const uint64_t* plane_busy,
                                 const uint64_t* plane_tags, const uint64_t* channel_cursor,
                                 uint64_t sequence, uint64_t burst_state)
{
    if (c == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(c->mu);
    const int st = ensure_engine(c);
    if (st != HBFSIM_OK) {
        return st;
    }
    return hbfamd::engine_set_state(c->eng, plane_busy, plane_tags, channel_cursor, sequence,
                                    burst_state);
}

HBF_API int hbfsim_amd_reset(hbfsim_context* c)
{
    if (c == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(c->mu);
    std::memset(&c->total, 0, sizeof(c->total));
    std::memset(&c->stats, 0, sizeof(c->stats));
    if (c->eng == nullptr) {
        return HBFSIM_OK;
    }
    return hbfamd::engine_reset(c->eng);
}

HBF_API int hbfsim_amd_last_kernel_ms(const hbfsim_context* c, float* ms, int max_kernels)
{
    if (c == nullptr || ms == nullptr || max_kernels <= 0) {
        return 0;
    }
    if (c->eng == nullptr) {
        return 0;
    }
    return hbfamd::engine_last_kernel_ms(c->eng, ms, max_kernels);
}

HBF_API int hbfsim_amd_last_apply_waves(const hbfsim_context* c)
{
    if (c == nullptr || c->eng == nullptr) {
        return 0;
    }
    return hbfamd::engine_last_apply_waves(c->eng);
}

HBF_API int hbfsim_amd_lookup_range(hbfsim_context* c, uint64_t address, uint32_t bytes,
                                    uint32_t* kind, hbfsim_amd_range* out, uint32_t* count)
{
    if (kind != nullptr) {
        *kind = 0;
    }
    if (c == nullptr || kind == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(c->mu);
    if (count != nullptr) {
        *count = static_cast<uint32_t>(c->ranges.size());
    }
    if (bytes == 0 || c->ranges.empty()) {
        return HBFSIM_OK;
    }
    std::size_t lo = 0, hi = c->ranges.size();  // upper_bound on base
    while (lo < hi) {
        const std::size_t mid = (lo + hi) / 2;
        if (address < c->ranges[mid].base) {
            hi = mid;
        } else {
            lo = mid + 1;
        }
    }
    if (lo == 0) {
        return HBFSIM_OK;
    }
    const hbfamd::range_rec& r = c->ranges[lo - 1];
    if (address < r.base || address - r.base >= r.length) {
        return HBFSIM_OK;
    }
    if (out != nullptr) {
        out->base = r.base;
        out->length = r.length;
        out->file_offset = r.file_offset;
        out->range_id = r.range_id;
        out->mode = r.mode;
        out->permissions = r.permissions;
        out->stream_id = r.stream_id;
        out->page_bytes = r.page_bytes;
    }
    *kind = (bytes > UINT64_MAX - address || address + bytes > r.base + r.length) ? 2u : 1u;
    return HBFSIM_OK;
}

HBF_API int hbfsim_amd_gen_segment_lines(hbf_record32* d_records, size_t capacity,
                                         const uint64_t* d_segment_base, size_t nseg,
                                         uint64_t lines_per_segment, uint32_t line_bytes,
                                         uint64_t gap_ps, uint32_t issuers, uint64_t flags,
                                         void* stream)
{
    return hbfamd::gen_segment_lines(d_records, capacity, d_segment_base, nseg,
                                     lines_per_segment, line_bytes, gap_ps, issuers, flags,
                                     stream);
}

HBF_API int hbfsim_amd_gen_spans(hbf_record32* d_records, size_t capacity,
                                 const uint64_t* d_span_base, const uint64_t* d_span_first,
                                 const uint32_t* d_span_op, size_t nspan, uint64_t total,
                                 uint32_t line_bytes, uint64_t gap_ps, uint32_t issuers,
                                 void* stream)
{
    return hbfamd::gen_spans(d_records, capacity, d_span_base, d_span_first, d_span_op, nspan,
                             total, line_bytes, gap_ps, issuers, stream);
}

HBF_API int hbfsim_amd_media_servers(const uint64_t* d_now_ns, size_t n, uint32_t servers,
                                     uint64_t latency_ns, uint64_t* d_completion_ns,
                                     void* stream)
{
    return hbfamd::media_servers(d_now_ns, n, servers, latency_ns, d_completion_ns, stream);
}

HBF_API int hbfsim_amd_mqsim_admission(const uint64_t* d_arrival_ns, const uint64_t* d_bytes,
                                       size_t n, uint32_t queue_depth, uint64_t latency_ns,
                                       uint64_t bandwidth_bytes_per_s, uint64_t* d_admission_ns,
                                       uint64_t* d_completion_ns, void* stream)
{
    return hbfamd::mqsim_admission(d_arrival_ns, d_bytes, n, queue_depth, latency_ns,
                                   bandwidth_bytes_per_s, d_admission_ns, d_completion_ns, stream);
}

struct hbfsim_amd_sampler {
    hbfamd::sampler_state* state;
};

HBF_API int hbfsim_amd_sampler_create(uint32_t warmup_requests, double sample_rate,
                                      uint64_t seed, hbfsim_amd_sampler** out)
{
    if (out == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    *out = nullptr;
    hbfamd::sampler_state* st = nullptr;
    const int rc = hbfamd::sampler_create(warmup_requests, sample_rate, seed, &st);
    if (rc != HBFSIM_OK) {
        return rc;
    }
    *out = new (std::nothrow) hbfsim_amd_sampler{st};
    if (*out == nullptr) {
        hbfamd::sampler_destroy(st);
        return HBFSIM_INVALID_ARGUMENT;
    }
    return HBFSIM_OK;
}

HBF_API void hbfsim_amd_sampler_destroy(hbfsim_amd_sampler* sampler)
{
    if (sampler != nullptr) {
        hbfamd::sampler_destroy(sampler->state);
        delete sampler;
    }
}

HBF_API int hbfsim_amd_sampler_reference(hbfsim_amd_sampler* sampler,
                                         const hbfsim_amd_access_class* d_access,
                                         const uint64_t* d_sequence, uint64_t first_sequence,
                                         size_t n, uint8_t* d_flags, uint64_t* references,
                                         void* stream)
{
    if (sampler == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    return hbfamd::sampler_reference(sampler->state, d_access, d_sequence, first_sequence, n,
                                     d_flags, references, stream);
}

HBF_API int hbfsim_amd_calibrate(const hbfsim_amd_access_class* d_access,
                                 const uint64_t* d_latency_ns, size_t n,
                                 hbfsim_amd_calibration* d_rows, size_t max_rows, size_t* rows,
                                 void* stream)
{
    return hbfamd::calibrate(d_access, d_latency_ns, n, d_rows, max_rows, rows, stream);
}

HBF_API int hbfsim_amd_link_run(const hbfsim_amd_link_profile* profile, const uint64_t* d_first,
                                uint32_t links, const uint64_t* d_ready_ns,
                                const uint8_t* d_direction, size_t n, uint64_t* d_delivered_ns,
                                hbfsim_amd_link_counters* d_counters, void* stream)
{
    if (profile == nullptr || profile->struct_size != sizeof(hbfsim_amd_link_profile)) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    try {
        return hbfamd::link_run(*profile, d_first, links, d_ready_ns, d_direction, n,
                                d_delivered_ns, d_counters, stream);
    } catch (...) {
        return HBFSIM_IO_ERROR;
    }
}

HBF_API int hbfsim_amd_link_run_traced(const hbfsim_amd_link_profile* profile,
                                       const uint64_t* d_first, uint32_t links,
                                       const uint64_t* d_ready_ns, const uint8_t* d_direction,
                                       size_t n, uint64_t* d_delivered_ns,
                                       hbfsim_amd_link_counters* d_counters,
                                       hbfsim_amd_link_flit* d_flits, uint32_t flit_limit,
                                       void* stream)
{
    if (profile == nullptr || profile->struct_size != sizeof(hbfsim_amd_link_profile) ||
        d_flits == nullptr || flit_limit == 0) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    try {
        return hbfamd::link_run(*profile, d_first, links, d_ready_ns, d_direction, n,
                                d_delivered_ns, d_counters, stream, d_flits, flit_limit);
    } catch (...) {
        return HBFSIM_IO_ERROR;
    }
}

HBF_API int hbfsim_amd_validate_profile(const char* path, char* error, size_t error_bytes)
{
    if (error != nullptr && error_bytes != 0) {
        error[0] = '\0';
    }
    if (path == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    try {
        (void)hbfamd::load_profile(path);
        return HBFSIM_OK;
    } catch (const std::exception& e) {
        if (error != nullptr && error_bytes != 0) {
            std::snprintf(error, error_bytes, "%s", e.what());
        }
        return HBFSIM_INVALID_ARGUMENT;
    } catch (...) {
        return HBFSIM_INVALID_ARGUMENT;
    }
}
