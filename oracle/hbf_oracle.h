/*
 * hbf_oracle.h -- CPU restatement of HBFSim's per-access timing path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the HIP engine is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load or call it.  The product path (hbfsim_amd/)
 * never links, loads or falls back to it.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the SlugLab/HBFSim tree).  Where the reference leaves a
 * semantic open (the multi-resource engine), the restatement follows the
 * frozen specification in the repository design notes, and the docstring says
 * which reference special case it must reduce to.
 *
 * Pinning status (what checks each function; see tests/test_oracle_*.py):
 *   fast_hash / hybrid_reference_sample  KAT (device_helper_abi_test.cpp:73-75)
 *                                        + golden vectors from compiled cuh
 *   fast_transfer_ns / fast_service_ns   KAT (device_helper_abi_test.cpp:79-81,
 *                                        348-355) + golden vectors + closed form
 *   find_range_index .. media_descriptor KAT (device_helper_abi_test.cpp:87-135,
 *                                        371-446) + brute force + golden vectors
 *   empirical_*                          KAT (device_helper_abi_test.cpp:137-225)
 *                                        + golden vectors
 *   range_table_*                        KAT (range_table_test.cpp) + invariants
 *   stripe                               CWDP KAT (ucie_bank_layout_test.cpp:34-50)
 *                                        + bijection invariants; other 23 orders:
 *                                        invariants only (MQSim un-vendored)
 *   engine_run (multi-resource)          reduces to fast_model_run and to the
 *                                        Lindley recursion; brute-force event
 *                                        simulation on tiny inputs
 *   fast_model_run                       closed-form recurrence hbf_device.cu:895-910
 *                                        and 796-881; hand-computed cases
 *   pagebuf (K=2 lower-slot rule)        golden traces from compiled
 *                                        device_coalescer.cpp
 *   media_servers (k-server)             golden traces from the k-server rule
 *   sampler_run / calibrate              KAT (calibrator_test.cpp:18-26, 92-105)
 *                                        + compiled calibrator.cpp on random
 *                                        streams (flags and estimates equal)
 *   thermal_dense_step                   closed forms (thermal_tests.cpp:54-89)
 *                                        + golden temperatures from compiled
 *                                        thermal.cpp
 *   arrhenius                            closed form + reliability test
 *                                        assertion (test_system_models.py:12)
 */
#ifndef HBF_ORACLE_H
#define HBF_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar helpers (hbf_device.cuh) --------------------------------- */
uint64_t orc_fast_hash(uint64_t value);
int orc_hybrid_reference_sample(uint64_t sequence, uint32_t warmup,
                                uint64_t threshold, uint64_t key);
uint64_t orc_sample_threshold(double rate);
uint64_t orc_fast_transfer_ns(uint32_t bytes, uint64_t bandwidth);
uint64_t orc_fast_service_ns(uint64_t base_ns, uint32_t bytes,
                             uint64_t bandwidth);
uint64_t orc_saturating_add(uint64_t a, uint64_t b);
uint64_t orc_saturating_multiply(uint64_t a, uint32_t b);

/* ---- range records (hbf_device.cuh:105-117) ------------------------- */
typedef struct orc_range {
    uint64_t base;
    uint64_t length;
    uint64_t file_offset;
    uint32_t range_id;
    uint32_t mode;
    uint32_t permissions;
    uint32_t cache_policy;
    uint32_t stream_id;
    uint32_t flags;
    uint64_t page_bytes;
    uint64_t reserved1;
} orc_range;

typedef struct orc_media {
    uint64_t logical_address;
    uint32_t bytes;
    uint32_t valid;
} orc_media;

uint32_t orc_find_range_index(const orc_range* ranges, uint32_t count,
                              uint64_t address);
int orc_access_supported(const orc_range* range, uint64_t address,
                         uint32_t bytes, uint32_t operation);
int orc_range_overlaps(const orc_range* range, uint64_t address,
                       uint32_t bytes);
int orc_span_touches_any_range(const orc_range* ranges, uint32_t count,
                               uint64_t address, uint32_t bytes);
orc_media orc_media_descriptor(const orc_range* range, uint64_t address,
                               uint32_t bytes, uint32_t operation);

/* Classification of one access, following the resolver's order of checks
 * (hbf_device.cu:1081-1165). */
enum orc_status {
    ORC_MODELED = 0,     /* timed by the engine */
    ORC_BYPASS = 1,      /* outside every range: native address, no delay */
    ORC_UNSUPPORTED = 2  /* straddles a range, crosses a page, no permission */
};
/* Record operations beyond read (0) and write (1): a refresh of media page
 * `addr` (read out and programmed back; plane tR + tPROG, channel `bytes`),
 * valid only with the media flag and only in streams whose parameters set
 * media_records (the coupled run's merged stream); elsewhere an operation
 * above 1 is unsupported, as the resolver has it. */
#define ORC_OP_REFRESH 2u
#define ORC_STATUS_GROUPED 32u
#define ORC_GROUP_MAX 64u
#define ORC_FLAG_MEDIA 0x100u
uint32_t orc_classify(const orc_range* ranges, uint32_t count,
                      uint64_t address, uint64_t bytes, uint32_t operation,
                      uint32_t* range_index);

/* ---- empirical curve (hbf_device.cuh:959-1140) ----------------------- */
uint64_t orc_ceiling_scaled_delta(uint64_t delta, uint32_t offset,
                                  uint32_t span);
uint64_t orc_empirical_cumulative_ns(const uint32_t* pages,
                                     const uint64_t* cumulative,
                                     uint32_t count, uint32_t run_pages);
uint64_t orc_empirical_service_ns(const uint32_t* pages,
                                  const uint64_t* cumulative, uint32_t count,
                                  uint32_t run_pages);
/* returns valid; writes packed state and run pages */
int orc_update_empirical_burst(uint64_t previous, uint64_t page,
                               uint32_t operation, uint64_t* packed,
                               uint32_t* run_pages);
typedef struct orc_empirical {
    uint32_t flags;          /* 1 = enabled */
    uint32_t point_count;    /* must be 6 */
    uint32_t pages[6];
    uint64_t cumulative_ns[6];
    uint64_t program_latency_ns;
} orc_empirical;
int orc_empirical_control_valid(const orc_empirical* e);
/* returns valid; writes service, packed state and run pages */
int orc_empirical_request_service(const orc_empirical* e, uint64_t previous,
                                  uint64_t page, uint32_t operation,
                                  uint64_t* service_ns, uint64_t* packed,
                                  uint32_t* run_pages);

/* ---- host range registry (range_table.cpp:17-198) -------------------- */
#define ORC_RANGE_CAPACITY 32768u
typedef struct orc_range_table {
    orc_range* records;      /* capacity ORC_RANGE_CAPACITY, sorted by base */
    uint32_t count;
    uint32_t next_range_id;
    uint64_t next_file_offset;
    uint64_t page_bytes;
    uint64_t media_capacity;
} orc_range_table;
orc_range_table* orc_range_table_create(uint64_t page_bytes,
                                        uint64_t media_capacity);
void orc_range_table_destroy(orc_range_table* t);
/* returns an hbfsim_error code: 0 ok, 1 invalid argument, 5 unsupported */
int orc_range_table_add(orc_range_table* t, uint64_t base, uint64_t length,
                        uint32_t mode, uint32_t permissions,
                        uint32_t cache_policy, uint32_t stream_id);
int orc_range_table_remove(orc_range_table* t, uint64_t base);
/* 0 outside, 1 matched, 2 crosses boundary; *index set when not outside */
int orc_range_table_lookup(const orc_range_table* t, uint64_t address,
                           uint32_t bytes, uint32_t* index);

/* ---- striping (profile.hpp:51-77; bank_layout.cpp:48-72) ------------- */
/* axis ids: 0 channel, 1 way (chip), 2 die, 3 plane.  order[0] advances
 * fastest.  sizes indexed by axis id.  coords indexed by axis id. */
uint64_t orc_stripe(uint64_t page, const uint32_t order[4],
                    const uint32_t sizes[4], uint32_t coords[4]);
int orc_parse_scheme(const char* name, uint32_t order[4]);
uint64_t orc_hbf_media_lpa(uint64_t q, uint32_t module, uint32_t channels);
void orc_hbf_cold_read_bank(uint64_t lpa, uint32_t channels,
                            uint32_t core_dies, uint32_t banks,
                            uint32_t* channel, uint32_t* core_die,
                            uint32_t* bank, uint32_t* chip);

/* ---- multi-resource engine (frozen specification) ------------------- */
enum orc_model {
    ORC_MODEL_HBF = 0,             /* plane (max,+) + channel cursor */
    ORC_MODEL_FAST_SCALAR = 1,     /* hbf_device.cu:883-958 single tail */
    ORC_MODEL_FAST_EMPIRICAL = 2   /* hbf_device.cu:796-881 single tail */
};

typedef struct orc_engine_params {
    uint32_t model;
    uint32_t channels, ways, dies, planes;  /* geometry */
    uint32_t order[4];                       /* fastest-first axis ids */
    uint32_t page_shift;                     /* log2(page bytes) */
    uint32_t page_buffers;                   /* K in {0,1,2} */
    uint32_t plane_contention;               /* 1: planes serialise */
    uint32_t transfer_page;                  /* 1: charge page bytes */
    uint32_t program_every_write;            /* 1: tPROG on every write */
    uint32_t hybrid;                         /* 1: count hybrid samples */
    uint32_t hybrid_warmup;
    uint64_t hybrid_threshold;
    uint64_t read_ps, program_ps;            /* base latencies in ps */
    uint64_t xfer_num, xfer_den;             /* xfer_ps =                  */
    uint64_t xfer_quantum;                   /*   q * ceil(b*num/den)      */
    orc_empirical empirical;                 /* MODEL_FAST_EMPIRICAL only */
    uint64_t media_pages;                    /* device pages; 0 = no limit */
    uint32_t media_records;                  /* 1: accept refresh records */
    uint32_t warp_grouping;                  /* 1: flags >> 32 is a group id */
} orc_engine_params;

typedef struct orc_engine_state {
    uint64_t* plane_busy;     /* [planes_total] */
    uint64_t* plane_tag;      /* [planes_total * 2]: page+1, 0 empty */
    uint64_t* channel_cursor; /* [channels] (1 for fast models) */
    uint64_t* plane_busy_total;
    uint64_t* channel_busy_total;
    uint64_t burst_state;     /* empirical packed burst state */
    uint64_t modeled_sequence;/* modeled requests so far */
} orc_engine_state;

typedef struct orc_engine_report {
    uint64_t records, modeled, bypass, unsupported;
    uint64_t reads, writes, page_hits, programs, hybrid_sampled;
    uint64_t makespan_ps;
    uint64_t latency_sum_lo, latency_sum_hi;
    uint64_t latency_max_ps;
    uint64_t service_sum_ps;
    uint64_t grouped;         /* records that shared an earlier one's request */
} orc_engine_report;

typedef struct orc_record {
    uint64_t addr, bytes, issue_ps, flags;
} orc_record;

/* Runs records in (issue time, position) order: in input order when the
 * stream is issue-ordered, else from a copy sorted stably by issue_ps (the
 * order in which the reference's MQSim adapter serves staged arrivals,
 * mqsim_online.cpp:269-289), results written back to input positions.
 * issue = base_ps + record.issue_ps.
 * completion[i]: completion ps (bypass: issue; unsupported: UINT64_MAX).
 * status may be NULL.  Report accumulates (caller zeroes it).
 *
 * Warp grouping (p->warp_grouping, hbf_device.cu:1223-1231): consecutive
 * records with the same nonzero group id (flags >> 32) are the lanes of one
 * warp instruction; a modeled record whose (range, media page) an earlier
 * modeled record of its group already has shares that record's request: it
 * takes its completion and status ORC_STATUS_GROUPED and touches no
 * resource, page register or hybrid sequence number.  Returns 6 before
 * anything is timed when a group has more than 64 records or two issue
 * times. */
int orc_engine_run(const orc_engine_params* p, const orc_range* ranges,
                   uint32_t range_count, const orc_record* records, size_t n,
                   uint64_t base_ps, orc_engine_state* s, uint64_t* completion,
                   uint8_t* status, orc_engine_report* report);
/* Same, records split over `threads` OpenMP threads by plane/channel
 * ownership (only for ORC_MODEL_HBF).  Bit-identical to orc_engine_run. */
int orc_engine_run_parallel(const orc_engine_params* p,
                            const orc_range* ranges, uint32_t range_count,
                            const orc_record* records, size_t n,
                            uint64_t base_ps, orc_engine_state* s,
                            uint64_t* completion, uint8_t* status,
                            orc_engine_report* report, int threads);

/* ---- the reference's scalar fast model, verbatim recurrence ----------- */
/* hbf_device.cu:883-958 with time_scale 1: for each request i (in order)
 *   tail = max(tail, arrival) + xfer; target = max(arrival + base, tail)
 * targets[i] written; returns fast_modeled_ns sum. */
uint64_t orc_fast_model_scalar(const uint64_t* arrival_ns,
                               const uint32_t* operation, const uint32_t* bytes,
                               size_t n, uint64_t read_ns, uint64_t program_ns,
                               uint64_t bandwidth, uint64_t* tail_ns,
                               uint64_t* target_ns);

/* ---- hbf_trace_timing fast loop (hbf_trace_timing.cpp:181-233) -------- */
typedef struct orc_trace_event {
    uint64_t logical_address, bytes;
    uint32_t page_bytes, operation;
} orc_trace_event;
/* returns 0 ok, 64 invalid argument (bad event) */
int orc_trace_timing_fast(const orc_trace_event* events, size_t n,
                          uint64_t read_ns, uint64_t program_ns,
                          uint64_t bandwidth, uint64_t profile_page_bytes,
                          uint64_t capacity_bytes, uint64_t* submitted,
                          uint64_t* service_ns, uint64_t* clock_ns);

/* ---- MQSim adapter bandwidth cursor (mqsim_online.cpp:321-335) -------- */
uint64_t orc_bandwidth_cursor(uint64_t* cursor_ns, uint64_t arrival_ns,
                              uint64_t bytes, uint64_t bandwidth,
                              uint64_t media_completion_ns);

/* ---- page-buffer slot rule (device_coalescer.cpp:134-168) ------------- */
/* Sequential accesses on one bank, each completing before the next.  K
 * slots; hit when the page is cached; a miss fills the first empty slot,
 * else the lowest slot.  hits[i] written. */
void orc_pagebuf_sequence(const uint64_t* pages, size_t n, uint32_t slots,
                          uint8_t* hits);

/* ---- MQSim adapter admission (mqsim_online.cpp:266-376) --------------
 * The adapter over a fake media port (in the style of the reference's
 * FakeMedia, ucie_device_frontend_fake_test.cpp:14-66) that completes
 * request i latency_ns[i] after it is handed over.  Requests are staged and
 * their arrival events registered in (arrival, index) order (flush_staged);
 * an arrival finding queue_depth requests in the device waits in a FIFO
 * (submit_to_device); a completion applies the bandwidth cursor
 * (orc_bandwidth_cursor, in completion order), frees its slot and
 * re-registers waiting requests at the current time
 * (release_admission_slots).  Events at one time fire in the order they
 * were registered, as MQSim's event queue fires them.  Outputs per request:
 * the time it was handed to the media port, the port's completion and the
 * bounded completion.  Returns 0, or 1 for bandwidth 0 or n >= 2^32. */
int orc_mqsim_admission(const uint64_t* arrival_ns, const uint64_t* bytes,
                        const uint64_t* latency_ns, size_t n, uint32_t queue_depth,
                        uint64_t bandwidth, uint64_t* admission_ns, uint64_t* device_ns,
                        uint64_t* completion_ns);

/* ---- k-server busy-until (prefetch_model.cpp:22-50) ------------------ */
/* orc_mqsim_admission with this engine as the media port: request k's
 * pages are records[first[k] .. first[k + 1]) (first: n + 1 entries), timed
 * by orc_engine_run (state s carried) when the loop dispatches the request,
 * issued at that time (ns * 1000 ps); the device completion is the ceiling
 * in ns of their latest completion.  admission_ns, device_ns and
 * completion_ns (bounded by the cursor) per request. */
int orc_engine_admission(const orc_engine_params* p, const orc_range* ranges,
                         uint32_t range_count, const orc_record* records,
                         const uint64_t* first, size_t n, const uint64_t* arrival_ns,
                         const uint64_t* bytes, uint32_t queue_depth, uint64_t bandwidth,
                         orc_engine_state* s, uint64_t* admission_ns, uint64_t* device_ns,
                         uint64_t* completion_ns);
void orc_media_servers(const uint64_t* now_ns, size_t n, uint32_t servers,
                       uint64_t latency_ns, uint64_t* completion_ns);

/* simulate_prefetch (prefetch_model.cpp:116-186), MediaServers and
 * StagingBuffer (:22-100) for the policies without a random predictor:
 * policy 0 None, 1 NextPage.  stats[7] = total_ns, stall_ns,
 * demand_accesses, demand_misses, prefetch_hits, prefetch_issued,
 * prefetch_wasted.  Returns 0, or 1 for another policy / no memory. */
int orc_simulate_prefetch(const uint64_t* pages, size_t n, uint32_t policy,
                          uint32_t lead_distance, uint32_t buffer_pages,
                          uint32_t max_in_flight, uint64_t read_latency_ns,
                          uint64_t compute_ns_per_access, uint64_t* stats);

/* ---- hybrid sampler and calibrator (calibrator.cpp:67-138) ----------- */
typedef struct orc_access_class {
    uint32_t operation;
    uint32_t bytes;
    uint32_t queue_bucket;
    uint32_t locality_bucket;
} orc_access_class;

/* HybridSampler(warmup, rate, seed) then flags[i] = reference(sequence[i],
 * access[i]) for i in order, from an empty seen set.  Returns 0, 1 for a
 * rate the constructor rejects, 2 when memory runs out. */
int orc_sampler_run(uint32_t warmup, double sample_rate, uint64_t seed,
                    const orc_access_class* access, const uint64_t* sequence,
                    size_t n, uint8_t* flags);

typedef struct orc_calibration {
    orc_access_class access;
    uint64_t count, mean_ns, p50_ns, p95_ns, p99_ns;
    double log_mean, log_sigma;
} orc_calibration;

/* Calibrator::observe(access[i], latency[i]) for all i, then estimate() of
 * every class observed, in the class order (std::map's).  Returns the row
 * count, or -1 for a zero latency (observe rejects it) or no memory. */
long orc_calibrate(const orc_access_class* access, const uint64_t* latency,
                   size_t n, orc_calibration* rows);

/* ---- thermal (thermal.cpp:127-311) ----------------------------------- */
/* One backward-Euler step of the RC network with constant power:
 * (C/dt + Gb + L) T' = C/dt T + Ps + E/dt + Gb Tb.  Dense Cholesky.
 * edges: pairs (a,b) with conductance g.  Returns 0 ok, 1 not SPD. */
int orc_thermal_dense_step(size_t n, const double* capacity,
                           const double* boundary_g, const double* boundary_t,
                           const double* static_power, size_t n_edges,
                           const uint32_t* edge_a, const uint32_t* edge_b,
                           const double* edge_g, double dt,
                           const double* energy, double* temperature);
/* Same step for a regular nx*ny*nz grid with 6-neighbour conductances gx,
 * gy, gz, uniform capacity, boundary conductance gb to tb on the top layer
 * (z = nz-1) only, power[n] watts; solved by Jacobi to |dT|<=tol or
 * max_sweeps.  Returns sweeps used. */
int orc_thermal_grid_step(uint32_t nx, uint32_t ny, uint32_t nz,
                          double capacity, double gx, double gy, double gz,
                          double gb, double tb, double dt,
                          const double* power, double* temperature,
                          double tol, int max_sweeps);
double orc_arrhenius(double temperature_k, double ea_ev, double tref_k);

/* ---- thermal-coupled reliability ------------------------------------ */
/* The EQ3 grid of orc_thermal_grid_step stepped once per window of
 * `window_ps` with a fixed number of Jacobi sweeps; power per cell from the
 * per-die access counts of the window (observer.cpp:42-72's energy per
 * window); per-die equivalent age advanced with the Arrhenius factor of the
 * die's hotspot (reliability.py:17-23, 93-108) through an integer lookup
 * table; refresh due when the age reaches the retention period
 * (cpu_service.cpp:169-217, the fixed period replaced by the derated one);
 * throttle level from the stack hotspot with hysteresis
 * (cpu_service.cpp:221-255).  Dies sit on the grid as follows: channel-way
 * q = c*W + w covers the x-y block (q % regions_x, q / regions_x); die d of
 * it covers layers [d*nz/D, (d+1)*nz/D). */
typedef struct orc_reliability {
    uint32_t nx, ny, nz, sweeps;
    double capacity, gx, gy, gz, gb, ambient_k, dt_s;
    uint64_t window_ps;
    uint32_t regions_x, regions_y, dies, policy; /* policy 1: hysteresis */
    double static_w;              /* W per cell */
    double access_energy_j, refresh_energy_j;
    double activation_ev, reference_k;
    uint64_t retention_ps;        /* refresh period at reference_k */
    double light_k, severe_k, shutdown_k, hysteresis_k;
    uint64_t action_delay_ps, min_dwell_ps, light_gap_ps;
} orc_reliability;

#define ORC_NO_PENDING 4u
typedef struct orc_control {
    uint32_t applied;  /* 0 none, 1 light, 2 severe, 3 shutdown */
    uint32_t pending;  /* ORC_NO_PENDING or the level waiting to apply */
    uint64_t pending_at_ps, last_change_ps;
} orc_control;

typedef struct orc_coupled_report {
    uint64_t windows, refreshes, deferred;
    uint64_t level_windows[4];
    uint64_t demand_modeled;
    uint64_t latency_sum_lo, latency_sum_hi, latency_max_ps;
    uint64_t makespan_ps;
    double peak_k;
} orc_coupled_report;

/* Retention lookup: table[b] = llround(window_ps * AF(T_b)), T_b = T0 +
 * (b + 1/2) / 16 K; bin(T) = floor((T - T0) * 16) clamped. */
#define ORC_AF_BINS 4096u
#define ORC_AF_T0 200.0
#define ORC_AF_STEPS_PER_K 16.0
void orc_retention_table(double ea_ev, double tref_k, uint64_t window_ps,
                         uint64_t* table);
uint32_t orc_retention_bin(double t);
/* One control sample at `now` with stack hotspot hs (cpu_service.cpp:
 * 221-255: control_sample, then apply_controls); returns the applied level. */
uint32_t orc_control_step(const orc_reliability* r, orc_control* c,
                          uint64_t now, double hs);
/* counts [windows][dies]; hot [(windows+1)][dies] (row 0 = initial);
 * level [windows]; refresh [windows][dies].  temperature, age and ctl are
 * updated in place. */
int orc_reliability_chain(const orc_reliability* r, const uint32_t* counts,
                          uint64_t windows, double* temperature, uint64_t* age,
                          orc_control* ctl, double* hot, uint8_t* level,
                          uint8_t* refresh);
/* First time >= t whose window's level is below `limit` (t itself when
 * its window allows; window starts otherwise). */
uint64_t orc_defer(const uint8_t* level, uint64_t windows, uint64_t window_ps,
                   uint64_t t, uint32_t limit);
/* Admission (cpu_service.cpp:256-285 for record streams): severe and
 * shutdown windows defer a request to the next window that admits demand;
 * light windows space admissions by light_gap_ps. */
void orc_admit(const uint8_t* level, uint64_t windows, uint64_t window_ps,
               uint64_t light_gap_ps, const orc_record* rec, size_t n,
               uint64_t* admit);
/* Refresh records (op 2, media flag) in (window, die) order; ordinal[die]
 * counts each die's refreshes and picks plane k % P and row k / P. */
size_t orc_refresh_records(const orc_engine_params* p, const uint8_t* refresh,
                           const uint8_t* level, uint64_t windows,
                           uint64_t window_ps, uint64_t* ordinal,
                           orc_record* out);
/* Merge by admission time, refresh records first on ties. */
void orc_merge_records(const orc_record* demand, const uint64_t* admit,
                       size_t n, const orc_record* extra, size_t r,
                       orc_record* out, uint64_t* demand_pos);
/* Modeled accesses per (window of issue_ps, die). */
int orc_window_counts(const orc_engine_params* p, const orc_range* ranges,
                      uint32_t range_count, const orc_record* rec, size_t n,
                      uint64_t window_ps, uint64_t windows, uint32_t* counts);
/* Thread count of the oracle's OpenMP parts (omp_set_num_threads): the
 * parallel engine's callers pass their own count; the Jacobi sweeps, the
 * hotspot reduction, the window counts and the coupled run's engine use
 * this one.  Results do not depend on it. */
void orc_set_threads(int threads);
int orc_get_threads(void);
/* The whole coupled run: counts -> chain -> admission -> refresh records ->
 * merge -> engine; completion[n] of the demand records.  hot, level and
 * refresh are sized for windows_cap windows.  Demand records must be in
 * issue order (1 otherwise, before anything changes). */
int orc_coupled_run(const orc_engine_params* p, const orc_range* ranges,
                    uint32_t range_count, const orc_reliability* r,
                    const orc_record* rec, size_t n, double* temperature,
                    uint64_t* age, orc_engine_state* s, uint64_t* completion,
                    orc_coupled_report* rep, double* hot, uint8_t* level,
                    uint8_t* refresh, uint64_t windows_cap);

/* ---- UCIe Streaming / AoU link (ucie_link.c; src/ucie/link.cpp) ------ */
typedef struct orc_link_profile {
    uint32_t gt_per_second;        /* 8, 16 or 32 (x64 lanes, Format 6) */
    uint32_t initial_ar_granules;  /* request-direction sender credits */
    uint32_t initial_r_granules;   /* return-direction sender credits */
    uint32_t max_accepted;         /* in-flight messages per direction */
    uint64_t propagation_ns;
} orc_link_profile;
typedef struct orc_link_counters {
    uint64_t flits, wire_bytes, ucie_header_bytes, crc_position_bytes;
    uint64_t aou_header_bytes, aou_message_bytes, unused_message_bytes;
    uint64_t credit_only_flits;
    uint64_t accounting_saturated;  /* 1 once any count reached 2^64 - 1 */
} orc_link_counters;
typedef struct orc_link_fragment {
    uint64_t request_id;
    uint32_t flit_granule, message_granule, granules;
    uint8_t msg_start, msg_end, pad[2];
} orc_link_fragment;
typedef struct orc_link_flit {
    uint32_t direction;            /* 0 request (AR), 1 return (R) */
    uint32_t nfrag;
    uint64_t start_ns, delivered_ns;
    uint32_t message_granules, grant_granules, credit_only, pad;
    orc_link_fragment frag[48];
} orc_link_flit;
typedef struct orc_link_delivery {
    uint32_t direction;
    uint32_t pad;
    uint64_t request_id;
    uint64_t delivered_ns;
} orc_link_delivery;
typedef struct orc_link orc_link;
int orc_link_profile_valid(const orc_link_profile* p);
uint64_t orc_link_serialization_ns(const orc_link_profile* p);
uint32_t orc_link_legal_grant(uint32_t pending);
orc_link* orc_link_create(const orc_link_profile* p);
void orc_link_destroy(orc_link* l);
int orc_link_enqueue(orc_link* l, uint32_t dir, uint64_t id, uint64_t ready_ns);
int orc_link_consume(orc_link* l, uint32_t dir, uint64_t id, uint64_t at);
int orc_link_next_event(const orc_link* l, uint64_t* t);
int orc_link_step(orc_link* l, orc_link_delivery* out, size_t cap, size_t* count);
uint64_t orc_link_now(const orc_link* l);
uint32_t orc_link_credits(const orc_link* l, uint32_t dir);
const orc_link_counters* orc_link_counters_of(const orc_link* l, uint32_t dir);
size_t orc_link_flit_count(const orc_link* l);
const orc_link_flit* orc_link_flit_at(const orc_link* l, size_t i);
int orc_link_scenario(const orc_link_profile* p, const uint32_t* dir, const uint64_t* ready,
                      size_t n, const uint64_t delay[2], uint64_t* delivered,
                      orc_link_counters* counters);
/* the same, also copying the link's flit records (the first 4096 in
 * emission order) to flits[0 .. min(count, flits_cap)) and the number not
 * recorded to *dropped */
int orc_link_scenario_traced(const orc_link_profile* p, const uint32_t* dir,
                             const uint64_t* ready, size_t n, const uint64_t delay[2],
                             uint64_t* delivered, orc_link_counters* counters,
                             orc_link_flit* flits, size_t flits_cap, size_t* nflits,
                             uint64_t* dropped);

#ifdef __cplusplus
}
#endif
#endif
