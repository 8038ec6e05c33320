// nes_launch.h -- host-side launchers for the kernels in nes_kernels.hip, and the
// error message shared by every C entry point.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "nes_layout.h"

namespace nesle {

// stats_mode: 0 none, 1 per-console counters, 2 counters + opcode/PC histograms.
// The auto-reset after a step is a separate launch_reset (below).
hipError_t launch_step(const DeviceState& s, std::uint32_t frameskip, std::uint32_t max_instr, int stats_mode,
                       hipStream_t stream);
// Masked (null = all) reset from the snapshot bank, or power-on without one.
// The auto-reset after a step is this launch with the step's done flags as
// the mask.
hipError_t launch_reset(const DeviceState& s, const std::uint8_t* mask, hipStream_t stream);
hipError_t launch_load_blob(const DeviceState& s, const std::uint8_t* blob_src, const std::uint8_t* mask,
                            hipStream_t stream);
hipError_t launch_save_blob(const DeviceState& s, std::uint32_t env, std::uint8_t* out, hipStream_t stream);
hipError_t launch_ram_obs(const DeviceState& s, std::uint8_t* obs, hipStream_t stream);
hipError_t launch_actions_i64(std::uint8_t* dst, const long long* src, std::uint32_t n, hipStream_t stream);
hipError_t launch_poke_ram(const DeviceState& s, std::uint32_t addr, std::uint32_t value, hipStream_t stream);
// One RAM byte per console: values[env] (device, n bytes) into RAM[addr].
hipError_t launch_poke_ram_envs(const DeviceState& s, std::uint32_t addr, const std::uint8_t* values,
                                hipStream_t stream);
hipError_t launch_seed_baselines(const DeviceState& s, hipStream_t stream);
// n 64-bit words set to zero by a kernel (graph-capturable, unlike a memset).
hipError_t launch_zero_u64(unsigned long long* p, std::uint32_t n, hipStream_t stream);
// Presentation snapshot (and pre-render latch) from live state, masked.
hipError_t launch_seed_present(const DeviceState& s, const std::uint8_t* mask, hipStream_t stream);
// Records of every console's live state (present::kHeader + vram_stride bytes
// each) into `out`, for a render of live state; the snapshot is untouched.
hipError_t launch_live_records(const DeviceState& s, std::uint8_t* out, hipStream_t stream);

// The ROM-less synthetic batch: masked (null = all, which also clears
// rewards, dones and step counts) power-on, and one env-step (pad applied
// or not) scored by the SMB rule.
hipError_t launch_synthetic_reset(const DeviceState& s, const std::uint8_t* mask, std::uint32_t* step_counts,
                                  hipStream_t stream);
hipError_t launch_synthetic_step(const DeviceState& s, std::uint32_t frameskip, std::uint32_t* step_counts,
                                 bool apply_actions, hipStream_t stream);

// The calling thread's message for nesle_last_error(), from entry points
// outside the batch (nes_host.hip keeps it).
void set_last_error(const std::string& msg);

}  // namespace nesle
