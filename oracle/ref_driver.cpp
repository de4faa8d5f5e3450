// ref_driver.cpp -- TEST INFRASTRUCTURE ONLY.
//
// A thin extern "C" shim over the reference's own dependency-free sources,
// compiled where they lie under the reference tree by oracle/Makefile's `ref`
// target into oracle/_ref/libhbfref.so.  It is used to pin the CPU oracle and
// to write golden vectors under tests/golden/; it is never part of the
// product and never shipped.  Only the reference's headers are included; no
// reference source is copied.
#include "src/cuda_runtime/device/hbf_device.cuh"

#include <hbfsim/eq3_thermal/thermal.hpp>
#include <hbfsim/hybrid_model.hpp>
#include <hbfsim/prefetch_model.hpp>
#include <hbfsim/ucie/bank_layout.hpp>
#include <hbfsim/ucie/device_coalescer.hpp>

#include <cstdint>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

#define REF_API extern "C" __attribute__((visibility("default")))

using hbfsim::device::SharedRangeRecord;

REF_API std::uint64_t ref_fast_hash(std::uint64_t v)
{
    return hbfsim::device::fast_hash(v);
}

REF_API int ref_hybrid_reference_sample(std::uint64_t seq, std::uint32_t warm,
                                        std::uint64_t thr, std::uint64_t key)
{
    return hbfsim::device::hybrid_reference_sample(seq, warm, thr, key);
}

REF_API std::uint64_t ref_fast_transfer_ns(std::uint32_t bytes,
                                           std::uint64_t bw)
{
    return hbfsim::device::fast_transfer_ns(bytes, bw);
}

REF_API std::uint64_t ref_fast_service_ns(std::uint64_t base,
                                          std::uint32_t bytes,
                                          std::uint64_t bw)
{
    return hbfsim::device::fast_service_ns(base, bytes, bw);
}

// calibrator.cpp:33-65 (host mirror)
REF_API std::uint64_t ref_host_fast_service_ns(std::uint64_t read_ns,
                                               std::uint64_t program_ns,
                                               std::uint64_t bw,
                                               std::uint32_t op,
                                               std::uint32_t bytes)
{
    const hbfsim::FastModelProfile profile{read_ns, program_ns, bw};
    const hbfsim::AccessClass access{
        op ? hbfsim::RequestOperation::Write : hbfsim::RequestOperation::Read,
        bytes, 0, 0};
    return hbfsim::fast_service_ns(profile, access);
}

// Range records are passed as the 64-byte SharedRangeRecord layout.
REF_API std::uint32_t ref_find_range_index(const SharedRangeRecord* r,
                                           std::uint32_t count,
                                           std::uint64_t addr)
{
    return hbfsim::device::find_range_index(r, count, addr);
}

REF_API int ref_access_supported(const SharedRangeRecord* r,
                                 std::uint64_t addr, std::uint32_t bytes,
                                 std::uint32_t op)
{
    return hbfsim::device::access_supported(*r, addr, bytes, op);
}

REF_API int ref_range_overlaps(const SharedRangeRecord* r, std::uint64_t addr,
                               std::uint32_t bytes)
{
    return hbfsim::device::range_overlaps(*r, addr, bytes);
}

REF_API int ref_span_touches_any_range(const SharedRangeRecord* r,
                                       std::uint32_t count,
                                       std::uint64_t addr,
                                       std::uint32_t bytes)
{
    return hbfsim::device::span_touches_any_range(r, count, addr, bytes);
}

REF_API int ref_media_descriptor(const SharedRangeRecord* r,
                                 std::uint64_t addr, std::uint32_t bytes,
                                 std::uint32_t op, std::uint64_t* logical,
                                 std::uint32_t* out_bytes)
{
    const auto m = hbfsim::device::media_descriptor(*r, addr, bytes, op);
    *logical = m.logical_address;
    *out_bytes = m.bytes;
    return m.valid;
}

REF_API std::uint64_t ref_empirical_cumulative_ns(const std::uint32_t* pages,
                                                  const std::uint64_t* cum,
                                                  std::uint32_t count,
                                                  std::uint32_t run)
{
    return hbfsim::device::empirical_cumulative_ns(pages, cum, count, run);
}

REF_API std::uint64_t ref_empirical_service_ns(const std::uint32_t* pages,
                                               const std::uint64_t* cum,
                                               std::uint32_t count,
                                               std::uint32_t run)
{
    return hbfsim::device::empirical_service_ns(pages, cum, count, run);
}

REF_API int ref_update_empirical_burst(std::uint64_t prev, std::uint64_t page,
                                       std::uint32_t op, std::uint64_t* packed,
                                       std::uint32_t* run)
{
    const auto u = hbfsim::device::update_empirical_burst(prev, page, op);
    *packed = u.packed;
    *run = u.run_pages;
    return u.valid;
}

REF_API int ref_empirical_request_service(const std::uint32_t* pages,
                                          const std::uint64_t* cum,
                                          std::uint64_t program_ns,
                                          std::uint64_t prev,
                                          std::uint64_t page, std::uint32_t op,
                                          std::uint64_t* service,
                                          std::uint64_t* packed,
                                          std::uint32_t* run)
{
    hbfsim::device::SharedControlHeader h{};
    h.empirical_flags = 1;
    h.empirical_point_count = 6;
    h.program_latency_ns = program_ns;
    for (int i = 0; i < 6; ++i) {
        h.empirical_breakpoint_pages[i] = pages[i];
        h.empirical_cumulative_ns[i] = cum[i];
    }
    const auto r = hbfsim::device::empirical_request_service(h, prev, page, op);
    *service = r.service_ns;
    *packed = r.packed_state;
    *run = r.run_pages;
    return r.valid;
}

// bank_layout.cpp:48-72 (scenario fixture layouts allowed)
REF_API int ref_cold_read_bank(std::uint64_t lpa, std::uint32_t channels,
                               std::uint32_t ncdu, std::uint32_t banks,
                               std::uint32_t* channel, std::uint32_t* die,
                               std::uint32_t* bank, std::uint32_t* chip)
{
    try {
        const hbfsim::ucie::HbfBankLayout layout{channels, ncdu, banks, true};
        const auto b = hbfsim::ucie::hbf_cold_read_bank(lpa, layout);
        *channel = b.host_channel;
        *die = b.core_die;
        *bank = b.bank;
        *chip = b.native_chip;
        return 1;
    } catch (const std::exception&) {
        return 0;
    }
}

REF_API int ref_hbf_media_lpa(std::uint64_t q, std::uint32_t module,
                              std::uint32_t channels, std::uint64_t* lpa)
{
    try {
        const hbfsim::ucie::HbfBankLayout layout{channels, 1, 16, true};
        *lpa = hbfsim::ucie::hbf_media_lpa(q, module, layout);
        return 1;
    } catch (const std::exception&) {
        return 0;
    }
}

// device_coalescer.cpp:61-254 driven one access at a time on one bank with
// the buffer cache on: arrive; a miss is submitted, completed and consumed
// before the next access arrives.  hits[i] = buffer_hit of access i.
REF_API int ref_pagebuf_sequence(const std::uint64_t* pages, std::size_t n,
                                 std::uint8_t* hits)
{
    try {
        hbfsim::ucie::DeviceReadCoalescer coal(4, 8, true, 1, 1);
        for (std::size_t i = 0; i < n; ++i) {
            const hbfsim::ucie::DevicePageKey key{1, 1, 0, 0, 7, pages[i], 0, 0};
            const auto waiter = static_cast<std::uint64_t>(i + 1);
            const auto a = coal.arrive(waiter, key);
            if (!a) {
                return 0;
            }
            hits[i] = a->buffer_hit ? 1 : 0;
            if (!a->buffer_hit) {
                const auto starts = coal.take_submittable();
                if (starts.size() != 1) {
                    return 0;
                }
                (void)coal.complete(starts[0].token, true);
            }
            coal.consume(waiter);
        }
        return 1;
    } catch (const std::exception&) {
        return 0;
    }
}

// thermal.cpp: build a model from flat arrays and advance once by dt with a
// single activity spanning [0, dt] carrying energy[i] joules on node i.
REF_API int ref_thermal_step(std::size_t n, const double* capacity,
                             const double* initial, const double* static_power,
                             const double* boundary_g, const double* boundary_t,
                             std::size_t n_edges, const std::uint32_t* ea,
                             const std::uint32_t* eb, const double* eg,
                             const double* energy, std::uint32_t steps,
                             double dt, double* out)
{
    using namespace hbfsim::eq3_thermal;
    try {
        ThermalModelConfig config;
        for (std::size_t i = 0; i < n; ++i) {
            ThermalNode node;
            node.id = "n" + std::to_string(i);
            node.physical_type = PhysicalType::Hbf;
            node.logical_role = LogicalRole::CapacityMemory;
            node.heat_capacity_j_per_k = capacity[i];
            node.initial_temperature_k = initial[i];
            node.static_power_w = static_power[i];
            node.boundary_conductance_w_per_k = boundary_g[i];
            node.boundary_temperature_k = boundary_t[i];
            config.nodes.push_back(node);
        }
        for (std::size_t e = 0; e < n_edges; ++e) {
            config.edges.push_back({ea[e], eb[e], eg[e],
                                    ConductanceKind::IntraComponent});
        }
        ThermalModel model(config);
        for (std::uint32_t s = 0; s < steps; ++s) {
            PhysicalActivity a;
            a.activity_id = s + 1;
            a.request_id = "step" + std::to_string(s);
            a.kind = ActivityKind::Read;
            a.start_time_s = dt * s;
            a.end_time_s = dt * (s + 1);
            a.completion_time_s = a.end_time_s;
            bool any = false;
            for (std::size_t i = 0; i < n; ++i) {
                if (energy != nullptr && energy[i] > 0.0) {
                    a.node_energy.push_back({i, energy[i]});
                    any = true;
                }
            }
            if (any) {
                model.add_activity(a);
            }
            model.advance_to(dt * (s + 1));
        }
        const auto& t = model.temperatures_k();
        std::memcpy(out, t.data(), n * sizeof(double));
        return 1;
    } catch (const std::exception&) {
        return 0;
    }
}

// simulate_prefetch (src/prefetch/prefetch_model.cpp:116-186): stats[7] =
// total_ns, stall_ns, demand_accesses, demand_misses, prefetch_hits,
// prefetch_issued, prefetch_wasted.
REF_API int ref_simulate_prefetch(const std::uint64_t* pages, std::size_t n, std::uint32_t policy,
                                  double accuracy, std::uint32_t lead_distance,
                                  std::uint32_t buffer_pages, std::uint32_t max_in_flight,
                                  std::uint64_t read_latency_ns, std::uint64_t compute_ns,
                                  std::uint64_t seed, std::uint64_t* stats)
{
    try {
        hbfsim::PrefetchConfig c;
        c.policy = static_cast<hbfsim::PrefetchPolicy>(policy);
        c.accuracy = accuracy;
        c.lead_distance = lead_distance;
        c.buffer_pages = buffer_pages;
        c.max_in_flight = max_in_flight;
        c.read_latency_ns = read_latency_ns;
        c.compute_ns_per_access = compute_ns;
        c.seed = seed;
        const std::vector<std::uint64_t> stream(pages, pages + n);
        const hbfsim::PrefetchStats r = hbfsim::simulate_prefetch(stream, c);
        stats[0] = r.total_ns;
        stats[1] = r.stall_ns;
        stats[2] = r.demand_accesses;
        stats[3] = r.demand_misses;
        stats[4] = r.prefetch_hits;
        stats[5] = r.prefetch_issued;
        stats[6] = r.prefetch_wasted;
        return 1;
    } catch (const std::exception&) {
        return 0;
    }
}

// HybridSampler (calibrator.cpp:67-96) over a stream: flags[i] =
// reference(sequence[i], access[i]) in order.  access holds n x 4 u32
// (operation, bytes, queue_bucket, locality_bucket).  Returns 1, or 0 when
// the constructor throws.
REF_API int ref_sampler_run(std::uint32_t warmup, double rate, std::uint64_t seed,
                            const std::uint32_t* access, const std::uint64_t* sequence,
                            std::size_t n, std::uint8_t* flags)
{
    try {
        hbfsim::HybridSampler sampler(warmup, rate, seed);
        for (std::size_t i = 0; i < n; ++i) {
            const hbfsim::AccessClass c{static_cast<hbfsim::RequestOperation>(access[4 * i]),
                                        access[4 * i + 1], access[4 * i + 2], access[4 * i + 3]};
            flags[i] = sampler.reference(sequence[i], c) ? 1 : 0;
        }
        return 1;
    } catch (const std::exception&) {
        return 0;
    }
}

// Calibrator (calibrator.cpp:98-136): observe every (access[i], latency[i]),
// then estimate(query).  out_u64 = count, mean, p50, p95, p99; out_f64 =
// log_mean, log_sigma.  Returns 1 with an estimate, 0 without one, -1 when
// observe throws.
REF_API int ref_calibrate(const std::uint32_t* access, const std::uint64_t* latency,
                          std::size_t n, const std::uint32_t* query, std::uint64_t* out_u64,
                          double* out_f64)
{
    try {
        hbfsim::Calibrator cal;
        for (std::size_t i = 0; i < n; ++i) {
            const hbfsim::AccessClass c{static_cast<hbfsim::RequestOperation>(access[4 * i]),
                                        access[4 * i + 1], access[4 * i + 2], access[4 * i + 3]};
            cal.observe(c, latency[i]);
        }
        const hbfsim::AccessClass q{static_cast<hbfsim::RequestOperation>(query[0]), query[1],
                                    query[2], query[3]};
        const auto e = cal.estimate(q);
        if (!e) {
            return 0;
        }
        out_u64[0] = e->count;
        out_u64[1] = e->mean_ns;
        out_u64[2] = e->p50_ns;
        out_u64[3] = e->p95_ns;
        out_u64[4] = e->p99_ns;
        out_f64[0] = e->log_mean;
        out_f64[1] = e->log_sigma;
        return 1;
    } catch (const std::exception&) {
        return -1;
    }
}
