// thermal.hpp -- host interface of the EQ3 thermal grid and the
// thermal-coupled reliability run (no HIP types).
#pragma once

#include "engine.hpp"

#include <cstddef>
#include <cstdint>

namespace hbfamd {

struct thermal;

int thermal_create(const hbfsim_amd_thermal_grid& grid, thermal** out);
void thermal_destroy(thermal* th);
const hbfsim_amd_thermal_grid& thermal_get_grid(const thermal* th);
// `steps` backward-Euler steps of the grid with constant power (W per
// cell), temperature in place.  Device pointers.
int thermal_step(thermal* th, const double* d_power, double* d_temperature,
                 std::uint64_t steps, void* stream);
// Average device time of one step's kernel in the last thermal_step call.
float thermal_last_step_ms(const thermal* th);
// Kernel passes the last thermal_step call launched (a pass makes one step,
// or two on the marching kernel's fused form).
std::uint64_t thermal_last_launches(const thermal* th);

// The coupled run on engine `e` (whose geometry `cfg` describes):
// per-window access counts -> thermal / retention / throttle chain ->
// admission -> refresh records -> merge -> engine run -> demand completions.
int coupled_run(engine* e, const engine_config& cfg, thermal* th,
                const hbfsim_amd_reliability_options& opt, const hbf_record32* d_records,
                std::size_t n, std::uint64_t* d_completion, double* d_temperature,
                std::uint64_t* age_ps, void* stream, hbfsim_amd_coupled_report* out,
                hbfsim_amd_report* engine_report);
// Device time (ms) of the last coupled run's phases: [0] access counts,
// [1] thermal chain, [2] admission and merge, [3] engine, [4] gather.
int coupled_last_ms(const thermal* th, float* ms, int max);
// Per-window trace of the last coupled run (host arrays).
int coupled_trace(const thermal* th, double* hot, std::size_t hot_count, std::uint8_t* level,
                  std::size_t level_count, std::uint8_t* refresh, std::size_t refresh_count,
                  std::uint64_t* windows, std::uint32_t* dies);

// Per-(window, die) counts of modeled records by issue time (engine.hip).
int engine_window_counts(engine* e, const hbf_record32* d_records, std::size_t n,
                         std::uint64_t window_ps, std::uint64_t windows,
                         std::uint32_t* d_counts, void* stream);

}  // namespace hbfamd
