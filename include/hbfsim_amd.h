/*
 * hbfsim_amd.h -- C ABI of the MI355X (gfx950) HBF access-timing engine.
 *
 * One shared library, hbfsim_amd/libhbfsim_amd.so, exports three groups of
 * entry points:
 *
 *   1. The reference's public C API, same names, argument meaning and error
 *      codes (include/hbfsim/api.h:12-107 in SlugLab/HBFSim).
 *   2. The reference's vLLM extension ABI (adapters/vllm/hbfsim_extension.h:
 *      10-26), ABI version 2, which the loader binds through ctypes
 *      (adapters/vllm/hbfsim_loader.py:287-385).
 *   3. Batch entry points that replace the reference's per-access device
 *      resolver (src/cuda_runtime/device/hbf_device.cu:765-959, 963-1344):
 *      a stream of access records in HBM is classified, striped and timed by
 *      HIP kernels, and completion timestamps come back in HBM.
 *
 * Plain C types only: no torch, no HIP types in any signature.  Device
 * pointers are plain addresses; streams are passed as `void*` (a hipStream_t,
 * NULL for the default stream).  Every function returns an hbfsim_error code
 * and never throws.
 */
#ifndef HBFSIM_AMD_H
#define HBFSIM_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ===== 1. Reference public API (include/hbfsim/api.h) ================== */

typedef struct hbfsim_context hbfsim_context;

/* api.h:12-20 */
enum hbfsim_error {
    HBFSIM_OK = 0,
    HBFSIM_INVALID_ARGUMENT = 1,
    HBFSIM_IO_ERROR = 2,
    HBFSIM_CUDA_ERROR = 3, /* here: any HIP runtime failure */
    HBFSIM_TIMEOUT = 4,
    HBFSIM_UNSUPPORTED = 5,
    HBFSIM_DAEMON_LOST = 6
};

/* api.h:22-40 */
enum hbfsim_range_mode {
    HBFSIM_RANGE_MODE_TIMING = 1,
    HBFSIM_RANGE_MODE_CAPACITY = 2
};
enum hbfsim_range_permission {
    HBFSIM_RANGE_READ = 1u << 0,
    HBFSIM_RANGE_WRITE = 1u << 1,
    HBFSIM_RANGE_READ_WRITE = HBFSIM_RANGE_READ | HBFSIM_RANGE_WRITE
};
enum hbfsim_cache_policy { HBFSIM_CACHE_POLICY_NONE = 0 };
enum hbfsim_model_mode {
    HBFSIM_MODEL_REFERENCE = 0,
    HBFSIM_MODEL_FAST = 1,
    HBFSIM_MODEL_HYBRID = 2
};

/* api.h:43-49 */
typedef struct hbfsim_options {
    const char* profile_path;
    const char* report_dir;
    uint32_t mode;
    uint32_t ring_capacity;
    uint64_t request_timeout_ns;
} hbfsim_options;

/* api.h:51-56 */
typedef struct hbfsim_range_options {
    uint32_t mode;
    uint32_t permissions;
    uint32_t cache_policy;
    uint32_t stream_id;
} hbfsim_range_options;

/* api.h:58-64 */
typedef struct hbfsim_stats {
    uint64_t requests_submitted;
    uint64_t requests_completed;
    uint64_t fast_requests;
    uint64_t reference_requests;
    uint64_t fast_modeled_ns;
} hbfsim_stats;

/* api.h:66-90 */
#define HBFSIM_CAPACITY_STATS_V1_VERSION 1u
typedef struct hbfsim_capacity_stats_v1 {
    uint32_t struct_size;
    uint32_t version;
    uint32_t enabled;
    uint32_t reserved0;
    uint64_t page_bytes;
    uint64_t vmm_granularity;
    uint64_t pool_allocated_bytes;
    uint64_t logical_frame_count;
    uint64_t service_resolve_calls;
    uint64_t service_resident_hits;
    uint64_t service_reclaimed_hits;
    uint64_t service_misses;
    uint64_t successful_backing_read_pages;
    uint64_t successful_backing_read_bytes;
    uint64_t successful_h2d_fill_pages;
    uint64_t successful_h2d_fill_bytes;
    uint64_t successful_resolve_evictions;
    uint64_t service_ready_results;
    uint64_t successful_d2h_readback_pages;
    uint64_t successful_d2h_readback_bytes;
    uint64_t successful_backing_write_pages;
    uint64_t successful_backing_write_bytes;
} hbfsim_capacity_stats_v1;

/* api.h:92 (src/api.cpp:3-6): returns 1 */
uint32_t hbfsim_abi_version(void);
/* api.h:93 (context.cpp:863-1000, 424-433): loads and validates the JSON
 * profile; ring_capacity must be a power of two in [2, 4096]; mode 0
 * (reference, needs the MQSim daemon) returns HBFSIM_UNSUPPORTED. */
int hbfsim_context_create(const hbfsim_options* options, hbfsim_context** out);
/* api.h:94 (context.cpp:1658-1717, range_table.cpp:17-118): registers a
 * TIMING range; CAPACITY ranges return HBFSIM_UNSUPPORTED. */
int hbfsim_register_device(hbfsim_context* context, void* device_ptr,
                           size_t length, const hbfsim_range_options* options);
/* api.h:97 (context.cpp:1719-1760): capacity mode is not part of this
 * engine; validates arguments, then returns HBFSIM_UNSUPPORTED. */
int hbfsim_map_file(hbfsim_context* context, const char* path,
                    uint64_t file_offset, size_t length,
                    const hbfsim_range_options* options,
                    void** logical_device_ptr_out);
/* api.h:101: waits for all engine work issued on the context */
int hbfsim_flush(hbfsim_context* context);
/* api.h:102 (context.cpp:1940-2007) */
int hbfsim_get_stats(hbfsim_context* context, hbfsim_stats* out);
/* api.h:103: capacity mode disabled -> zeros with enabled = 0 */
int hbfsim_get_capacity_stats_v1(hbfsim_context* context,
                                 hbfsim_capacity_stats_v1* out);
/* api.h:105 (context.cpp:2063-2110, range_table.cpp:120-171) */
int hbfsim_unregister(hbfsim_context* context, void* range_base);
/* api.h:106 */
void hbfsim_context_destroy(hbfsim_context* context);

/* ===== 2. vLLM extension ABI (adapters/vllm/hbfsim_extension.h) ======== */

typedef struct hbfsim_vllm_session hbfsim_vllm_session;

/* hbfsim_extension.h:12-18 */
typedef struct hbfsim_vllm_options {
    const char* profile_path;
    const char* report_dir;
    uint32_t ring_capacity;
    uint32_t timing_model;
    uint64_t request_timeout_ns;
} hbfsim_vllm_options;

/* hbfsim_extension.cpp:13-16: returns 2 */
uint32_t hbfsim_vllm_abi_version(void);
/* hbfsim_extension.cpp:18-49 */
int hbfsim_vllm_session_create(const hbfsim_vllm_options* options,
                               hbfsim_vllm_session** out);
/* hbfsim_extension.cpp:51-67: TIMING range with READ permission */
int hbfsim_vllm_register_storage(hbfsim_vllm_session* session,
                                 uintptr_t device_address, size_t bytes);
/* hbfsim_extension.cpp:69-81: nulls *session */
int hbfsim_vllm_session_close(hbfsim_vllm_session** session);
/* hbfsim_extension.cpp:83-101 */
const char* hbfsim_vllm_status_string(int status);
/* No counterpart in the reference: the engine context behind a session, so
 * a vLLM worker can run the batch engine on the ranges it registered. */
hbfsim_context* hbfsim_vllm_session_context(hbfsim_vllm_session* session);

/* ===== 3. Batch timing engine ========================================== */

/* One access record, 32 bytes, 16-byte aligned.  Replaces one call of the
 * reference's per-access resolver __hbfsim_resolve(addr, bytes, op)
 * (hbf_device.cu:963).  issue_ps is the issue time in picoseconds relative
 * to the run's base_ps.  flags bits 0-7: operation (0 read, 1 write); bits
 * 32-63: warp group id (0: none), read when the engine option
 * warp_grouping is 1; other bits are ignored.  A record's service order on
 * every resource is its place in (issue time, stream position) order: its
 * stream position when records are ordered by issue time (the fast case),
 * else its position in the stably sorted stream (see hbfsim_amd_run_device).
 * The thermal-coupled run also merges refresh records into the
 * stream it times: operation 2 with flag bit 8 set, addr = media page, bytes
 * moved on the channel (read out and written back); elsewhere operation 2
 * is unsupported like any operation above 1.
 *
 * Warp grouping (hbf_device.cu:1223-1231): the reference resolves the
 * active lanes of one warp instruction together, and lanes that passed
 * validation and touch the same (range, page) share one media request, that
 * of the lowest lane.  Here the lanes of one instruction are consecutive
 * records with the same nonzero group id (at most 64, one issue time); a
 * modeled record whose (range, page) an earlier modeled record of its group
 * already has takes that record's completion, consumes no plane, channel or
 * page register, takes no hybrid sequence number, and reports status
 * HBFSIM_AMD_STATUS_GROUPED.  With warp_grouping 0 (the default) every record
 * is its own request, which equals the reference when the caller passes one
 * record per (warp instruction, range, page). */
typedef struct hbf_record32 {
    uint64_t addr;
    uint64_t bytes;
    uint64_t issue_ps;
    uint64_t flags;
} hbf_record32;

/* Packed 16-byte record, an input format of this engine with no
 * counterpart in the reference: half the bytes of hbf_record32 per access
 * for the hot path.  addr_bytes holds the address in bits 0-47 and the byte
 * count in bits 48-63; issue_op holds issue_ps in bits 0-55 and the
 * operation (0 read, 1 write) in bits 56-63.  It carries every record whose
 * address is below 2^48, byte count below 2^16, issue time below 2^56 ps and
 * flags below 256 (no refresh records). */
typedef struct hbf_record16 {
    uint64_t addr_bytes;
    uint64_t issue_op;
} hbf_record16;

/* Per-record status byte: bits 0-1 class (0 modeled, 1 bypass: outside
 * every range, 2 unsupported: rejected by the resolver's checks), bit 2
 * page-buffer hit, bit 3 selected by the hybrid sampler, bit 4 write that
 * programmed the page, bit 5 modeled record that shared an earlier record's
 * media request (warp grouping). */
enum hbfsim_amd_status_bits {
    HBFSIM_AMD_MODELED = 0,
    HBFSIM_AMD_BYPASS = 1,
    HBFSIM_AMD_UNSUPPORTED = 2,
    HBFSIM_AMD_PAGE_HIT = 4,
    HBFSIM_AMD_HYBRID_SAMPLED = 8,
    HBFSIM_AMD_PROGRAMMED = 16,
    HBFSIM_AMD_STATUS_GROUPED = 32
};

enum hbfsim_amd_model {
    /* planes serialise tR / tPROG with a per-plane page buffer; channels
     * are bandwidth cursors in issue order; completion is the later of the
     * two (the reference's latency-overlaps-transfer rule,
     * hbf_device.cuh:797-816, per resource) */
    HBFSIM_AMD_MODEL_HBF = 0,
    /* the reference's empirical single-tail model, hbf_device.cu:796-881:
     * burst runs of consecutive pages price reads on the profile's
     * cumulative curve; profiles with empirical_vmem and 4 KiB pages */
    HBFSIM_AMD_MODEL_EMPIRICAL = 1
};

/* Engine configuration beyond the reference profile.  The reference profile
 * schema forbids extra keys, so these travel separately.  Zero-initialised
 * fields take the documented defaults. */
typedef struct hbfsim_amd_engine_options {
    uint32_t struct_size;          /* sizeof(hbfsim_amd_engine_options) */
    uint32_t model;                /* hbfsim_amd_model */
    uint32_t page_buffers;         /* page registers per plane: 0, 1, 2 (2: a miss
                                      fills the first empty slot, else slot 0) */
    uint32_t plane_contention;     /* 1: planes serialise their service */
    uint32_t transfer_page;        /* 1: channel moves the whole page */
    uint32_t program_every_write;  /* 1: every write pays tPROG */
    uint32_t flat_geometry;        /* 1: one channel, one plane */
    uint32_t ways;                 /* chips per channel (default 1) */
    uint64_t xfer_quantum_ps;      /* transfer rounded up to this (1) */
    uint64_t channel_bandwidth_bytes_per_s; /* 0: aggregate / channels */
    uint32_t tile_records;         /* records per tile, multiple of 64;
                                      0 chooses per run (default) */
    uint32_t warp_grouping;        /* 1: records with a group id share media
                                      requests (32-byte records, HBF model,
                                      at most one page register) */
} hbfsim_amd_engine_options;

/* Result of one run (or, from hbfsim_amd_get_report, of all runs). */
typedef struct hbfsim_amd_report {
    uint64_t records;
    uint64_t modeled;
    uint64_t bypass;
    uint64_t unsupported;
    uint64_t reads;
    uint64_t writes;
    uint64_t page_hits;
    uint64_t programs;
    uint64_t hybrid_sampled;
    uint64_t makespan_ps;      /* latest completion of a modeled record */
    uint64_t latency_sum_lo;   /* sum of completion - issue, 128 bits */
    uint64_t latency_sum_hi;
    uint64_t latency_max_ps;
    uint64_t service_sum_ps;   /* sum of uncontended service times */
    uint64_t grouped;          /* modeled records that shared an earlier
                                  record's media request (warp grouping);
                                  counted in records, modeled, reads/writes
                                  and the latencies, not in page_hits,
                                  programs, hybrid_sampled or service_sum_ps */
} hbfsim_amd_report;

/* Defaults: HBF model (EMPIRICAL when the profile carries empirical_vmem),
 * one page register per plane, planes serialise, access-sized transfers. */
int hbfsim_amd_default_engine_options(const hbfsim_context* context,
                                      hbfsim_amd_engine_options* out);
/* Replaces the engine configuration; resets engine state. */
int hbfsim_amd_set_engine_options(hbfsim_context* context,
                                  const hbfsim_amd_engine_options* options);
int hbfsim_amd_get_engine_options(const hbfsim_context* context,
                                  hbfsim_amd_engine_options* out);

/* Time n records resident in device memory (the hot path).  completion_ps
 * [n] (device) receives completion times: issue for bypass records,
 * UINT64_MAX for unsupported ones.  status [n] (device) may be NULL.
 * base_ps is added to every issue_ps.  Engine state (per-plane busy and
 * page-buffer tags, per-channel cursors) carries over from the previous run
 * on the context.  `report` (host) may be NULL.  The call returns when the
 * run has completed on `stream`.
 *
 * Order: every resource serves its records in (issue time, position) order,
 * as the reference's MQSim adapter serves staged arrivals sorted by
 * (arrival, sequence) (mqsim_online.cpp:269-289).  An issue-ordered stream
 * is timed as it lies; when some record's issue time is below its
 * predecessor's, the run leaves the engine state untouched, times a copy of
 * the records sorted stably by issue time (allocating about 40 bytes per
 * record more) and writes completions and status bytes back to the records'
 * positions; the hybrid sampler's sequence numbers follow the sorted order.
 * Up to 2^32 - 1 records per run in that case (HBFSIM_UNSUPPORTED beyond). */
int hbfsim_amd_run_device(hbfsim_context* context,
                          const hbf_record32* records, size_t n,
                          uint64_t* completion_ps, uint8_t* status,
                          uint64_t base_ps, void* stream,
                          hbfsim_amd_report* report);
/* hbfsim_amd_run_device for packed records: the same results as the
 * 32-byte records they pack.  Contexts with two page registers or the
 * empirical model return HBFSIM_UNSUPPORTED. */
int hbfsim_amd_run_device_packed(hbfsim_context* context,
                                 const hbf_record16* records, size_t n,
                                 uint64_t* completion_ps, uint8_t* status,
                                 uint64_t base_ps, void* stream,
                                 hbfsim_amd_report* report);
/* hbfsim_amd_run_device_packed for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference.  Same arguments and
 * results; it calls no allocator: the run's scratch (per tile of T records:
 * 64 B per plane, 24 B per channel, 16 B per 64 planes and 145 B; per group
 * of 16 tiles the same summaries; 16 B per 64 records) comes from a static
 * array of 64 MiB per device, held until the process ends.  T is the
 * context's tile_records or, by default, the automatic tile doubled (up to
 * 16,384) until the run fits: up to about 125 million records per call with
 * 64 planes and 8 channels, 27 million with 512 planes and 16 channels and
 * 13 million with 1,024 planes and 256 channels.  Returns
 * HBFSIM_UNSUPPORTED, touching neither the context nor *report,
 * when the run does not fit, when the context's engine does not exist yet
 * (make one ordinary run first), when ranges were registered or removed
 * since the last run (the range upload allocates), in hybrid mode, or when
 * the static array's device address cannot be looked up.  It cannot sort:
 * records whose issue time goes back return HBFSIM_INVALID_ARGUMENT with the
 * context and *report untouched (completion_ps and status then hold no
 * result).  Every call on a device shares that device's array: calls that
 * overlap on one device race. */
int hbfsim_amd_run_device_packed_noalloc(hbfsim_context* context,
                                         const hbf_record16* records, size_t n,
                                         uint64_t* completion_ps, uint8_t* status,
                                         uint64_t base_ps, void* stream,
                                         hbfsim_amd_report* report);
/* Same with host buffers: copies in, runs on the default stream, copies
 * out. */
int hbfsim_amd_run(hbfsim_context* context, const hbf_record32* records,
                   size_t n, uint64_t* completion_ps, uint8_t* status,
                   uint64_t base_ps, hbfsim_amd_report* report);
/* Cumulative report over every run since the last reset. */
int hbfsim_amd_get_report(const hbfsim_context* context,
                          hbfsim_amd_report* out);
/* Geometry the engine uses: planes = channels*ways*dies*planes_per_die. */
int hbfsim_amd_get_geometry(const hbfsim_context* context, uint32_t* channels,
                            uint32_t* planes);
/* Per-resource busy totals (ps of service charged), cumulative.  Host
 * arrays of at least `planes` and `channels` entries (either may be NULL). */
int hbfsim_amd_get_busy_totals(hbfsim_context* context, uint64_t* plane_ps,
                               size_t planes, uint64_t* channel_ps,
                               size_t channels);
/* Engine state for checkpoint / resume: plane busy [planes], plane page tags
 * [planes * 2] (page + 1, 0 empty), channel cursors [channels], plus the
 * modeled-request sequence and the empirical burst state.  Host arrays. */
int hbfsim_amd_get_state(hbfsim_context* context, uint64_t* plane_busy,
                         uint64_t* plane_tags, uint64_t* channel_cursor,
                         uint64_t* sequence, uint64_t* burst_state);
int hbfsim_amd_set_state(hbfsim_context* context, const uint64_t* plane_busy,
                         const uint64_t* plane_tags,
                         const uint64_t* channel_cursor, uint64_t sequence,
                         uint64_t burst_state);
/* Zeroes engine state, busy totals and the cumulative report. */
int hbfsim_amd_reset(hbfsim_context* context);
/* Average device time (ms) of each engine kernel over the last run,
 * measured with HIP events on the run's stream: [0] tile summary, [1] carry
 * chain, [2] apply.  Returns the number of kernels written. */
int hbfsim_amd_last_kernel_ms(const hbfsim_context* context, float* ms,
                              int max_kernels);
/* Diagnostics, no counterpart in the reference: the waves per SIMD the last
 * run's apply kernel was built for (4: the form for large streams of general
 * steps, taken when the engine's previous run of at least 2^24 records had
 * fewer page-register hits than an eighth of its modeled records; 3: packed
 * records otherwise; 1: 32-byte records, two page registers or refresh
 * records), 0 before any run and after an empirical-model run (no apply
 * pass).  Results do not depend on the form. */
int hbfsim_amd_last_apply_waves(const hbfsim_context* context);

/* One registered range as the registry holds it (SharedRangeRecord,
 * hbf_device.cuh:105-117). */
typedef struct hbfsim_amd_range {
    uint64_t base;
    uint64_t length;
    uint64_t file_offset;
    uint32_t range_id;
    uint32_t mode;
    uint32_t permissions;
    uint32_t stream_id;
    uint64_t page_bytes;
} hbfsim_amd_range;

/* RangeTable::lookup (range_table.cpp:173-198): *kind = 0 outside every
 * range, 1 matched, 2 crosses the range end; `out` filled unless outside.
 * Also returns the number of registered ranges in *count (may be NULL). */
int hbfsim_amd_lookup_range(hbfsim_context* context, uint64_t address,
                            uint32_t bytes, uint32_t* kind,
                            hbfsim_amd_range* out, uint32_t* count);

/* Workload compiler, no counterpart in the reference (it generates the
 * record streams the benchmark configurations describe).  Writes
 * nseg * lines_per_segment records to d_records (device, capacity
 * records): segment s, line k -> addr = d_segment_base[s] + k * line_bytes,
 * bytes = line_bytes, issue_ps = (index / issuers) * gap_ps, flags.  The
 * records are ordered by issue time.  Asynchronous on `stream`. */
int hbfsim_amd_gen_segment_lines(hbf_record32* d_records, size_t capacity,
                                 const uint64_t* d_segment_base, size_t nseg,
                                 uint64_t lines_per_segment, uint32_t line_bytes,
                                 uint64_t gap_ps, uint32_t issuers, uint64_t flags,
                                 void* stream);

/* Workload compiler for spans of different lengths, no counterpart in the
 * reference (it generates the TinyLlama weight-streaming and paged-KV
 * configurations).  Span s covers records [d_span_first[s],
 * d_span_first[s + 1]) (nspan + 1 device entries, starting at 0 and ending
 * at total <= capacity, non-decreasing): line k of the span reads (op 0) or
 * writes (op 1) line_bytes at d_span_base[s] + k * line_bytes; record j is
 * issued at (j / issuers) * gap_ps.  Asynchronous on `stream`. */
int hbfsim_amd_gen_spans(hbf_record32* d_records, size_t capacity,
                         const uint64_t* d_span_base, const uint64_t* d_span_first,
                         const uint32_t* d_span_op, size_t nspan, uint64_t total,
                         uint32_t line_bytes, uint64_t gap_ps, uint32_t issuers, void* stream);

/* MediaServers::issue (src/prefetch/prefetch_model.cpp:22-50) for a batch:
 * `servers` identical servers (0 counts as 1), all free at time 0, each read
 * taking latency_ns; read i, issued at d_now_ns[i], starts when the
 * earliest-free server frees (or at its issue time) and completes
 * latency_ns later, in d_completion_ns[i].  Device arrays of n entries.
 * Issue times must not decrease (simulate_prefetch's clock never runs
 * backwards, prefetch_model.cpp:124-186) and must stay below 2^63 ns:
 * HBFSIM_INVALID_ARGUMENT otherwise (completions are then unspecified).
 * Synchronises `stream`. */
int hbfsim_amd_media_servers(const uint64_t* d_now_ns, size_t n, uint32_t servers,
                             uint64_t latency_ns, uint64_t* d_completion_ns, void* stream);

/* The MQSim adapter's queue-depth admission and bandwidth cursor
 * (mqsim_online.cpp:291-376: submit_to_device, dispatch_to_device, the
 * completion callback, release_admission_slots) over a media port that
 * completes every request latency_ns after it is handed over (the role of
 * MQSim, which is not part of this engine).  Requests in submission order
 * with non-decreasing d_arrival_ns; at most max(1, queue_depth) are in the
 * device at a time, the rest wait in arrival order; each completion applies
 * cursor = max(cursor, arrival) + ceil(bytes * 1e9 / bandwidth).
 * d_admission_ns[i] (may be NULL): when request i was handed over;
 * d_completion_ns[i]: max(admission + latency, cursor), the adapter's
 * bounded completion.  Device arrays; synchronises `stream`.
 * HBFSIM_INVALID_ARGUMENT for bandwidth 0, arrivals out of order or times
 * from 2^63 ns. */
int hbfsim_amd_mqsim_admission(const uint64_t* d_arrival_ns, const uint64_t* d_bytes, size_t n,
                               uint32_t queue_depth, uint64_t latency_ns,
                               uint64_t bandwidth_bytes_per_s, uint64_t* d_admission_ns,
                               uint64_t* d_completion_ns, void* stream);

/* ----- Hybrid model: request sampler and calibrator -------------------
 * The host-side HybridSampler and Calibrator of src/hybrid/calibrator.cpp
 * (include/hbfsim/hybrid_model.hpp:13-60) for batches of requests held in
 * device memory.  hbfsim_amd_access_class is AccessClass (operation 0 read,
 * 1 write) and orders like its defaulted operator<=>: operation, bytes,
 * queue_bucket, locality_bucket. */
typedef struct hbfsim_amd_access_class {
    uint32_t operation;
    uint32_t bytes;
    uint32_t queue_bucket;
    uint32_t locality_bucket;
} hbfsim_amd_access_class;

/* CalibrationEstimate (hybrid_model.hpp:28-36) with its class. */
typedef struct hbfsim_amd_calibration {
    hbfsim_amd_access_class access;
    uint64_t count;
    uint64_t mean_ns;
    uint64_t p50_ns;
    uint64_t p95_ns;
    uint64_t p99_ns;
    double log_mean;
    double log_sigma;
} hbfsim_amd_calibration;

typedef struct hbfsim_amd_sampler hbfsim_amd_sampler;

/* HybridSampler(warmup_requests, sample_rate, seed) (calibrator.cpp:67-81):
 * HBFSIM_INVALID_ARGUMENT for a rate outside [0, 1] or not finite (the
 * constructor's std::invalid_argument). */
int hbfsim_amd_sampler_create(uint32_t warmup_requests, double sample_rate, uint64_t seed,
                              hbfsim_amd_sampler** out);
void hbfsim_amd_sampler_destroy(hbfsim_amd_sampler* sampler);

/* HybridSampler::reference (calibrator.cpp:83-96) for n requests in order:
 * d_flags[i] = reference(sequence_i, d_access[i]), with sequence_i =
 * d_sequence[i], or first_sequence + i when d_sequence is NULL (the
 * consecutive sequences of hbf_trace_timing.cpp:181-206).  The sampler keeps
 * the classes it has seen across calls, as the reference's seen set does.
 * *references (if not NULL) receives the number of flags set.  Device
 * arrays; synchronises `stream`.  n must be below 2^32. */
int hbfsim_amd_sampler_reference(hbfsim_amd_sampler* sampler,
                                 const hbfsim_amd_access_class* d_access,
                                 const uint64_t* d_sequence, uint64_t first_sequence, size_t n,
                                 uint8_t* d_flags, uint64_t* references, void* stream);

/* Calibrator::observe(d_access[i], d_latency_ns[i]) for every i, then
 * estimate() of every class observed (calibrator.cpp:98-136), one row per
 * class in class order into d_rows.  count, mean_ns (floor of the 128-bit
 * sum / count) and the percentiles equal the reference's; log_mean and
 * log_sigma are computed in double on the GPU (the reference sums in long
 * double) and agree to 1e-12 relative.  *rows receives the class count;
 * HBFSIM_INVALID_ARGUMENT when it exceeds max_rows (nothing written) or
 * when a latency is 0 (observe's "latency_ns must be positive").  Device
 * arrays; synchronises `stream`.  n must be below 2^32. */
int hbfsim_amd_calibrate(const hbfsim_amd_access_class* d_access, const uint64_t* d_latency_ns,
                         size_t n, hbfsim_amd_calibration* d_rows, size_t max_rows,
                         size_t* rows, void* stream);

/* ===== 4. EQ3 thermal grid and thermal-coupled reliability =============
 *
 * The reference's RC network (src/eq3_thermal/thermal.cpp:127-311) on a
 * regular grid: nx * ny * nz cells (x fastest, z = nz - 1 the top layer),
 * uniform heat capacity, conductances gx / gy / gz between neighbouring
 * cells and top_g from every top-layer cell to the ambient.  One step is
 * ThermalModel::advance_to's backward-Euler solve,
 *   (C/dt + G_top + L) T' = C/dt T + P + G_top T_ambient,
 * by `sweeps` Jacobi sweeps (the system is strictly diagonally dominant;
 * at the stiffness of a 1-us step a few sweeps reach double precision). */
typedef struct hbfsim_amd_thermal_grid {
    uint32_t struct_size;      /* sizeof(hbfsim_amd_thermal_grid) */
    uint32_t nx, ny, nz;
    uint32_t sweeps;           /* Jacobi sweeps per step, 1..8 */
    uint32_t reserved0;
    double capacity_j_per_k;   /* per cell */
    double gx_w_per_k, gy_w_per_k, gz_w_per_k;
    double top_g_w_per_k;      /* each top-layer cell to ambient */
    double ambient_k;
    double dt_s;               /* step length */
} hbfsim_amd_thermal_grid;

typedef struct hbfsim_amd_thermal hbfsim_amd_thermal;

/* Replaces ThermalModel's constructor for a grid network
 * (thermal.cpp:242-311).  Owns device scratch on the current device.
 * HBFSIM_UNSUPPORTED for a grid that no kernel takes: steps run on staged
 * tiles of at most 2,048 cells ((t + 2 sweeps)^2 nz for some tile edge t),
 * or, on grids of at least 2^21 cells, on the marching kernel (at most 16
 * layers with 1-4 sweeps, at most 8 with 5-8; nx >= 2 (64 - 2 sweeps),
 * ny >= 8 sweeps). */
int hbfsim_amd_thermal_create(const hbfsim_amd_thermal_grid* grid,
                              hbfsim_amd_thermal** out);
/* ThermalModel::advance_to (thermal.cpp:127-160) with constant power:
 * `steps` steps.  d_power: W per cell; d_temperature: K per cell, updated in
 * place.  Device arrays of nx*ny*nz doubles.  Returns when done. */
int hbfsim_amd_thermal_step(hbfsim_amd_thermal* thermal, const double* d_power,
                            double* d_temperature, uint64_t steps,
                            void* stream);
/* Average device time (ms) of one step in the last hbfsim_amd_thermal_step
 * call, from HIP events on its stream. */
int hbfsim_amd_thermal_last_ms(const hbfsim_amd_thermal* thermal, float* ms);
/* Kernel passes the last hbfsim_amd_thermal_step call launched: one per step,
 * except that on the marching kernel with 1-4 sweeps one pass makes two steps
 * (the power is the same in both).  A diagnostic with no counterpart in the
 * reference: it turns last_ms into a per-pass time. */
int hbfsim_amd_thermal_last_launches(const hbfsim_amd_thermal* thermal, uint64_t* launches);
void hbfsim_amd_thermal_destroy(hbfsim_amd_thermal* thermal);

/* Thermal-coupled refresh and throttling.  The grid is stepped once per
 * window (window_ps = dt).  Channel-way q = c * ways + w occupies the x-y
 * block (q % regions_x, q / regions_x) of the grid; die d of it occupies
 * layers [d * nz / dies, (d + 1) * nz / dies).  Per window:
 *  - control (cpu_service.cpp:221-255, policy "hysteresis"): the stack
 *    hotspot sets the throttle level (0 none, 1 light, 2 severe,
 *    3 shutdown) through light/severe/shutdown thresholds, hysteresis,
 *    action delay and minimum dwell;
 *  - retention (reliability.py:17-23, 93-108; cpu_service.cpp:169-217):
 *    each die's equivalent age advances by window_ps times the Arrhenius
 *    factor of its hotspot, looked up in a table of 1/16-K bins from 200 K;
 *    at the retention period a refresh of one page of the die is issued
 *    (plane k % P, row k / P for the die's k-th refresh) and the age
 *    restarts;
 *  - power: static + access_energy * (modeled accesses issued to the die in
 *    the window) / dt + refresh_energy * refreshes / dt, spread evenly over
 *    the die's cells (observer.cpp:42-72).
 * Admission (cpu_service.cpp:256-285): records issued in severe or shutdown
 * windows wait for the next window that admits demand; in light windows
 * admissions are spaced by light_gap_ps; refreshes wait only for shutdown.
 * Refresh records (op 2, media flag) join the stream at their admission
 * time, before demand records admitted at the same time, and are timed by
 * the engine like any access (plane tR + tPROG, two pages on the channel). */
typedef struct hbfsim_amd_reliability_options {
    uint32_t struct_size;      /* sizeof(hbfsim_amd_reliability_options) */
    uint32_t policy;           /* 0 sample only, 1 hysteresis */
    uint32_t regions_x, regions_y;  /* regions_x * regions_y = channels*ways */
    uint64_t window_ps;        /* must equal the grid's dt */
    double static_power_w;     /* per cell */
    double access_energy_j;    /* per modeled access */
    double refresh_energy_j;   /* per refresh */
    double activation_energy_ev;
    double reference_k;        /* Arrhenius reference temperature */
    uint64_t retention_ps;     /* refresh period at reference_k */
    double light_k, severe_k, shutdown_k, hysteresis_k;
    uint64_t action_delay_ps, min_dwell_ps, light_gap_ps;
} hbfsim_amd_reliability_options;

typedef struct hbfsim_amd_coupled_report {
    uint64_t windows;
    uint64_t refreshes;
    uint64_t deferred;           /* demand records admitted after issue */
    uint64_t level_windows[4];   /* windows at each throttle level */
    uint64_t demand_modeled;
    uint64_t latency_sum_lo;     /* completion - issue over modeled demand */
    uint64_t latency_sum_hi;
    uint64_t latency_max_ps;
    uint64_t makespan_ps;        /* latest completion incl. refreshes */
    double peak_k;               /* hottest die hotspot of the run */
} hbfsim_amd_coupled_report;

/* One coupled run over n issue-ordered demand records (device), issue_ps
 * from time 0.  d_completion_ps [n] (device) receives the demand
 * completions; d_temperature (device, grid cells) holds the initial
 * temperature and receives the final one; age_ps (host, channels * ways *
 * dies entries) holds each die's equivalent age and is updated.  Engine
 * state carries over as for hbfsim_amd_run_device.  Either report may be
 * NULL; engine_report covers the merged stream.  Refused before anything
 * changes (temperature, ages, engine state): demand records whose issue time
 * goes back (HBFSIM_INVALID_ARGUMENT: the windows, the admission gate and
 * the merge follow issue order), and contexts with warp grouping or two
 * page registers (HBFSIM_UNSUPPORTED: the engine times the merged refresh
 * records only without them). */
int hbfsim_amd_run_coupled(hbfsim_context* context, hbfsim_amd_thermal* thermal,
                           const hbfsim_amd_reliability_options* options,
                           const hbf_record32* d_records, size_t n,
                           uint64_t* d_completion_ps, double* d_temperature,
                           uint64_t* age_ps, void* stream,
                           hbfsim_amd_coupled_report* report,
                           hbfsim_amd_report* engine_report);
/* Device time (ms) of the last coupled run's phases, from HIP events on its
 * stream: [0] access counts, [1] thermal chain (all windows), [2] admission
 * and merge, [3] engine on the merged stream, [4] gather.  Returns the
 * number written (-1 on a NULL argument). */
int hbfsim_amd_coupled_last_ms(const hbfsim_amd_thermal* thermal, float* ms,
                               int max_phases);
/* Per-window trace of the last coupled run: die hotspots [(windows + 1) *
 * dies] (row 0 = the initial temperature), throttle levels [windows],
 * refresh flags [windows * dies].  Host arrays (any may be NULL); counts are
 * checked.  *windows and *dies receive the sizes. */
int hbfsim_amd_coupled_trace(const hbfsim_amd_thermal* thermal, double* hot,
                             size_t hot_count, uint8_t* level, size_t level_count,
                             uint8_t* refresh, size_t refresh_count,
                             uint64_t* windows, uint32_t* dies);

/* ===== 5. UCIe Streaming / AoU link ====================================
 *
 * The reference's StreamingLink (src/ucie/link.cpp:1-203; profile rules of
 * src/ucie/profile.cpp:40-67) for batches of independent links, one link
 * per GPU thread.  A link carries AR requests (3 AoU granules, direction 0)
 * and R returns (14 granules, direction 1); each direction sends a Format 6
 * flit of 48 granules every 32 / GT ns while it has data or a credit grant
 * to send; a message's granules are all reserved against the sender's
 * credits at its MsgStart; credits come back as grants of 1, 4, 8, ... 128
 * granules riding flits of the other direction after the receiver consumes
 * the message.
 *
 * The link's caller (the reference leaves it to its user,
 * link.hpp:62-65) is fixed here: it admits each direction's messages in
 * order while fewer than max_accepted of that direction are in flight (the
 * reference's enqueue refuses more, link.cpp:45-46), at the later of the
 * message's ready time and the time it finds room, and consumes every
 * delivered message consume_delay_ns[direction] after its delivery. */
typedef struct hbfsim_amd_link_profile {
    uint32_t struct_size;          /* sizeof(hbfsim_amd_link_profile) */
    uint32_t gt_per_second;        /* 8, 16 or 32 (x64 lanes) */
    uint32_t initial_ar_granules;  /* 3..65535 */
    uint32_t initial_r_granules;   /* 14..65535 */
    uint32_t max_accepted;         /* 1..65535 in flight per direction */
    uint32_t reserved0;
    uint64_t propagation_ns;       /* at most 1e9 and (4094 flits in flight) */
    uint64_t consume_delay_ns[2];  /* [0] AR, [1] R */
} hbfsim_amd_link_profile;

/* DirectionCounters (link.hpp:41-50): each count is bounded at 2^64 - 1,
 * and accounting_saturated (0 or 1) says whether any reached the bound
 * (link.cpp:15-23). */
typedef struct hbfsim_amd_link_counters {
    uint64_t flits;
    uint64_t wire_bytes;
    uint64_t ucie_header_bytes;
    uint64_t crc_position_bytes;
    uint64_t aou_header_bytes;
    uint64_t aou_message_bytes;
    uint64_t unused_message_bytes;
    uint64_t credit_only_flits;
    uint64_t accounting_saturated;
} hbfsim_amd_link_counters;

/* FlitRecord and its Fragment (link.hpp:22-38).  request_id is the
 * message's position in its link plus one (the reference's ids are the
 * caller's, nonzero).  A Format 6 flit holds at most 16 fragments: 48
 * granules of 3-granule AR messages, or of at most 5 pieces of 14-granule R
 * messages. */
typedef struct hbfsim_amd_link_fragment {
    uint64_t request_id;
    uint32_t flit_granule;
    uint32_t message_granule;
    uint32_t granules;
    uint8_t msg_start;
    uint8_t msg_end;
    uint8_t reserved[2];
} hbfsim_amd_link_fragment;

typedef struct hbfsim_amd_link_flit {
    uint64_t start_ns;
    uint64_t delivered_ns;
    uint64_t step;                /* the link's event step that sent it (from 0) */
    uint32_t direction;           /* 0 AR (Request), 1 R (Return) */
    uint32_t message_granules;
    uint32_t grant_granules;
    uint32_t credit_only;         /* 0 or 1 */
    uint32_t fragments;           /* entries of fragment[] in use */
    uint32_t reserved;
    hbfsim_amd_link_fragment fragment[16];
} hbfsim_amd_link_flit;

/* Runs `links` links to quiescence.  Link l's messages are
 * [d_first[l], d_first[l + 1]) of d_ready_ns / d_direction (d_first has
 * links + 1 entries, from 0 to n); within a link each direction's ready
 * times must not decrease.  d_delivered_ns[i] receives message i's delivery
 * time; d_counters[2 * l + direction] the link's counters.  Device arrays;
 * synchronises `stream`.  HBFSIM_INVALID_ARGUMENT for a profile outside the
 * reference's rules, a direction above 1, ready times out of order or an
 * event time beyond 2^64 - 1 ns (the reference's overflow_error), a link of
 * 2^32 messages or more or malformed offsets; HBFSIM_UNSUPPORTED when more
 * than 4094 flits could be in flight.  The library keeps the scratch of its
 * largest call per device (12 B per message plus 12 B per flit slot and
 * link) until the process ends; calls on one device run one at a time. */
int hbfsim_amd_link_run(const hbfsim_amd_link_profile* profile, const uint64_t* d_first,
                        uint32_t links, const uint64_t* d_ready_ns,
                        const uint8_t* d_direction, size_t n, uint64_t* d_delivered_ns,
                        hbfsim_amd_link_counters* d_counters, void* stream);
/* hbfsim_amd_link_run that also records flits (StreamingLink::flits(),
 * link.cpp:150-156): d_flits[(2 * l + d) * flit_limit + k] receives link
 * l's k-th flit of direction d for k < min(flit_limit, that direction's
 * flits counter); later flits are counted but not recorded.  The
 * reference's single list per link is both directions' flits ordered by
 * step, the request direction first within a step (each direction sends at
 * most one flit per step; several steps can share an event time); its first
 * 4,096 flits, with the rest counted as flit_records_dropped, are recovered
 * from flit_limit = 4096.  The same refusals, plus HBFSIM_INVALID_ARGUMENT for d_flits null
 * or flit_limit 0. */
int hbfsim_amd_link_run_traced(const hbfsim_amd_link_profile* profile, const uint64_t* d_first,
                               uint32_t links, const uint64_t* d_ready_ns,
                               const uint8_t* d_direction, size_t n, uint64_t* d_delivered_ns,
                               hbfsim_amd_link_counters* d_counters, hbfsim_amd_link_flit* d_flits,
                               uint32_t flit_limit, void* stream);

/* Profile validation with the reference's rules and messages
 * (src/profile/profile.cpp:238-468).  Returns HBFSIM_OK or
 * HBFSIM_INVALID_ARGUMENT with the reference's message in `error`. */
int hbfsim_amd_validate_profile(const char* path, char* error,
                                size_t error_bytes);

/* ===== 6. Measurement ==================================================
 *
 * No counterpart in the reference: the HBM ceilings the benchmark prices
 * its per-record passes against, measured with their access patterns.
 * Streams `bytes` of d_buffer (device, 16-byte aligned, at least 256 KiB)
 * `reps` times with 16-byte non-temporal loads, one wave per 256 KiB and 16
 * loads in flight per lane (the summary pass's record stream), then `reps`
 * times with 16-byte non-temporal stores of whole 1 KiB rows, one wave per
 * 128 KiB (the apply pass's completion stream); *read_ms and *write_ms
 * receive the average time of one pass (HIP events on `stream`).  The
 * buffer's contents are overwritten.  Synchronises `stream`. */
int hbfsim_amd_probe_bandwidth(void* d_buffer, size_t bytes, unsigned reps, void* stream,
                               float* read_ms, float* write_ms);

#ifdef __cplusplus
}
#endif
#endif
