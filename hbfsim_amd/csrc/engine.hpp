// engine.hpp -- host interface of the HIP timing engine (no HIP types).
#pragma once

#include "../../include/hbfsim_amd.h"

#include <cstddef>
#include <cstdint>
#include <functional>
#include <vector>

namespace hbfamd {

// One registered range, the 64-byte SharedRangeRecord of the reference
// (hbf_device.cuh:105-117).
struct range_rec {
    std::uint64_t base;
    std::uint64_t length;
    std::uint64_t file_offset;
    std::uint32_t range_id;
    std::uint32_t mode;
    std::uint32_t permissions;
    std::uint32_t cache_policy;
    std::uint32_t stream_id;
    std::uint32_t flags;
    std::uint64_t page_bytes;
    std::uint64_t reserved1;
};
static_assert(sizeof(range_rec) == 64, "range record layout");

// Everything the kernels need, resolved from profile + engine options.
struct engine_config {
    std::uint32_t model{HBFSIM_AMD_MODEL_HBF};
    std::uint32_t channels{1}, ways{1}, dies{1}, planes{1};
    std::uint32_t order[4]{0, 1, 2, 3};  // fastest-first axis ids C W D P
    std::uint32_t page_shift{12};
    std::uint32_t slots{1};
    std::uint32_t contention{1};
    std::uint32_t transfer_page{0};
    std::uint32_t every_write{0};
    std::uint32_t hybrid{0};
    std::uint32_t hybrid_warmup{0};
    std::uint64_t hybrid_threshold{0};
    std::uint64_t read_ps{0}, program_ps{0};
    std::uint64_t xfer_num{1}, xfer_den{1}, xfer_quantum{1};
    std::uint32_t tile{4096};
    std::uint32_t grouping{0};         // warp grouping of records with a group id
    std::uint64_t media_pages{~0ull};  // device capacity in pages
    std::uint32_t emp_pages[6]{};
    std::uint64_t emp_cum_ns[6]{};
    std::uint64_t emp_program_ns{0};

    std::uint32_t n_channels() const { return channels; }
    std::uint32_t n_planes() const { return channels * ways * dies * planes; }
};

struct engine;

// Returns HBFSIM_OK or an error; *out owns device memory on the current
// device.
int engine_create(const engine_config& config, engine** out);
void engine_destroy(engine* e);
const engine_config& engine_get_config(const engine* e);
int engine_set_ranges(engine* e, const std::vector<range_rec>& ranges);
// refresh_records: the stream may hold refresh records (op 2 with the media
// flag); without it they are classified like any other operation > 1.
int engine_run(engine* e, const hbf_record32* d_records, std::size_t n,
               std::uint64_t* d_completion, std::uint8_t* d_status,
               std::uint64_t base_ps, void* stream, hbfsim_amd_report* out,
               bool refresh_records = false);
// The same for packed 16-byte records (main pipeline only: one page
// register, no hybrid sampling, HBF model; else HBFSIM_UNSUPPORTED).
int engine_run_packed(engine* e, const hbf_record16* d_records, std::size_t n,
                      std::uint64_t* d_completion, std::uint8_t* d_status,
                      std::uint64_t base_ps, void* stream, hbfsim_amd_report* out);
// engine_run_packed without allocating: the run's scratch comes from a
// static per-device array of kNoAllocScratchBytes.  HBFSIM_UNSUPPORTED when
// the run's scratch does not fit it (at the largest tile, 16,384 records), or
// when the range table changed since the last run (uploading it allocates).
constexpr std::size_t kNoAllocScratchBytes = std::size_t{64} << 20;
int engine_run_packed_noalloc(engine* e, const hbf_record16* d_records, std::size_t n,
                              std::uint64_t* d_completion, std::uint8_t* d_status,
                              std::uint64_t base_ps, void* stream, hbfsim_amd_report* out);
int engine_get_busy_totals(engine* e, std::uint64_t* plane_ps, std::size_t planes,
                           std::uint64_t* channel_ps, std::size_t channels);
int engine_get_state(engine* e, std::uint64_t* plane_busy, std::uint64_t* plane_tags,
                     std::uint64_t* channel_cursor, std::uint64_t* sequence,
                     std::uint64_t* burst);
int engine_set_state(engine* e, const std::uint64_t* plane_busy,
                     const std::uint64_t* plane_tags, const std::uint64_t* channel_cursor,
                     std::uint64_t sequence, std::uint64_t burst);
int engine_reset(engine* e);
int engine_synchronize(engine* e);
int engine_last_kernel_ms(const engine* e, float* ms, int max_kernels);
int engine_last_apply_waves(const engine* e);
// Host <-> device staging helpers for the host-pointer entry point.
int engine_run_host(engine* e, const hbf_record32* records, std::size_t n,
                    std::uint64_t* completion, std::uint8_t* status,
                    std::uint64_t base_ps, hbfsim_amd_report* out);

// Issue order (order.hip).  order_check sets *d_flag (device) to 1 when some
// record's issue time is below its predecessor's; asynchronous on `stream`.
int order_check(const void* d_records, bool packed, std::size_t n, std::uint32_t* d_flag,
                void* stream);
// Times a stream in (issue time, position) order: sorts a copy of the
// records stably by issue time, calls run(sorted records, completions,
// status) with device buffers in that order (status NULL when d_status is),
// then scatters completions and status bytes back to stream positions and
// synchronises `stream`.  HBFSIM_UNSUPPORTED from 2^32 records.
using sorted_runner =
    std::function<int(const void* d_sorted, std::uint64_t* d_comp, std::uint8_t* d_status)>;
int run_in_issue_order(const void* d_records, bool packed, std::size_t n,
                       std::uint64_t* d_completion, std::uint8_t* d_status, void* stream,
                       const sorted_runner& run);

// Workload compiler (gen.hip).
int gen_segment_lines(hbf_record32* d_records, std::size_t capacity,
                      const std::uint64_t* d_seg_base, std::size_t nseg, std::uint64_t lines,
                      std::uint32_t line_bytes, std::uint64_t gap_ps, std::uint32_t issuers,
                      std::uint64_t flags, void* stream);

// Variable-length spans of lines (gen.hip): d_first has nspan + 1 entries,
// d_first[0] = 0 and d_first[nspan] = total <= capacity (checked on the host).
int gen_spans(hbf_record32* d_records, std::size_t capacity, const std::uint64_t* d_base,
              const std::uint64_t* d_first, const std::uint32_t* d_op, std::size_t nspan,
              std::uint64_t total, std::uint32_t line_bytes, std::uint64_t gap_ps,
              std::uint32_t issuers, void* stream);

// k identical media servers (servers.hip).
int media_servers(const std::uint64_t* d_now, std::size_t n, std::uint32_t servers,
                  std::uint64_t latency_ns, std::uint64_t* d_completion, void* stream);

// hbfsim_amd_mqsim_admission (admission.hip).  Synchronises `stream`.
int mqsim_admission(const std::uint64_t* d_arrival, const std::uint64_t* d_bytes, std::size_t n,
                    std::uint32_t queue_depth, std::uint64_t latency_ns,
                    std::uint64_t bandwidth, std::uint64_t* d_admission,
                    std::uint64_t* d_completion, void* stream);

// Hybrid model's sampler and calibrator (hybrid.hip).
struct sampler_state;
int sampler_create(std::uint32_t warmup, double sample_rate, std::uint64_t seed,
                   sampler_state** out);
void sampler_destroy(sampler_state* s);
int sampler_reference(sampler_state* s, const hbfsim_amd_access_class* d_access,
                      const std::uint64_t* d_sequence, std::uint64_t first_sequence,
                      std::size_t n, std::uint8_t* d_flags, std::uint64_t* references,
                      void* stream);
int calibrate(const hbfsim_amd_access_class* d_access, const std::uint64_t* d_latency,
              std::size_t n, hbfsim_amd_calibration* d_rows, std::size_t max_rows,
              std::size_t* rows_out, void* stream);

}  // namespace hbfamd
