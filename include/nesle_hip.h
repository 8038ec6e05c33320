/* nesle_hip.h -- C ABI of libnesle_hip.so, the MI355X batched NROM console.
 *
 * Plain C: opaque handle, pointers and sizes, integer status codes.  Every
 * entry point replaces one piece of the reference's pybind11 binding
 * nesle._cuda_core (cpp/bindings/cuda_module.cu); the citation on each
 * declaration names the reference interface it stands in for.  The Python
 * drop-in (nesle_amd/_cuda_core, class CudaBatch) is a thin layer over these.
 *
 * Status codes: NESLE_OK, or NESLE_EINVAL for bad arguments (the reference's
 * std::invalid_argument -> ValueError) and NESLE_ERUNTIME / NESLE_EDEVICE for
 * parse and HIP failures (std::runtime_error -> RuntimeError).
 * nesle_last_error() returns the calling thread's last message.
 *
 * Threading and streams: calls on one handle must not overlap.  All device
 * work runs on the handle's stream (nesle_set_stream; default the null
 * stream, as the reference's launches are).  Entry points that return host
 * data synchronise that stream; nesle_step does not unless asked.
 */
#ifndef NESLE_HIP_H
#define NESLE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    NESLE_OK = 0,
    NESLE_EINVAL = 1,
    NESLE_ERUNTIME = 2,
    NESLE_EDEVICE = 3
};

/* Reward rules (applied once per env-step, after the last frame). */
enum {
    NESLE_REWARD_SMB = 0,    /* cpp/include/nesle/cuda/batch_step.cuh:61-106 */
    NESLE_REWARD_XDELTA = 1  /* clip(int16(x - x_prev), -clip, clip) - time_penalty;
                                done when RAM[done_addr] == 0; x = RAM[x_lo] | RAM[x_hi] << 8 */
};

/* Device views (nesle_get_view kinds). */
enum {
    NESLE_VIEW_RAM = 0,          /* uint8  [num_envs][2048], env-major      */
    NESLE_VIEW_REWARDS = 1,      /* float  [num_envs]                       */
    NESLE_VIEW_DONES = 2,        /* uint8  [num_envs]                       */
    NESLE_VIEW_ACTIONS = 3,      /* uint8  [num_envs]                       */
    NESLE_VIEW_INSTRUCTIONS = 4, /* uint64 [num_envs] (after stats steps)   */
    NESLE_VIEW_FRAMES = 5,       /* uint32 [num_envs] frames completed (after stats steps) */
    NESLE_VIEW_BUDGET_HITS = 6,  /* uint32 [num_envs]   (after stats steps) */
    NESLE_VIEW_OPCODES = 7,      /* uint64 [256]     (after profile steps)  */
    NESLE_VIEW_PCS = 8,          /* uint64 [65536]                          */
    NESLE_VIEW_OAM = 9,          /* uint8  [num_envs][256] (host copy only) */
    NESLE_VIEW_FRAME_RGB = 10,   /* uint8  [num_envs][240][256][3] (after nesle_render) */
    NESLE_VIEW_FRAME_PALETTE = 11, /* uint8 [num_envs][240][256] palette values 0-63 */
    NESLE_VIEW_GRAY84 = 12,      /* uint8  [num_envs][84][84] gray observation */
    NESLE_VIEW_CENSUS = 13,      /* uint64 [32] step-kernel census (after stats mode 3 steps) */
    NESLE_VIEW_PRESENT = 14,     /* uint8  [num_envs][16 + video memory block] presentation records:
                                    frame-start x, y, ctrl, frame-end x, y, ctrl, mask, 9 spare
                                    bytes, then palette, OAM and nametable RAM as frozen at the last
                                    vblank (what nesle_render draws); frames on only */
    NESLE_VIEW_COUNT = 15
};

/* nesle_render outputs (bit mask). */
enum {
    NESLE_FRAME_RGB = 1,
    NESLE_FRAME_PALETTE = 2,
    NESLE_FRAME_GRAY84 = 4,
    NESLE_FRAME_LIVE = 8    /* modifier: draw live state with the CPU core's rules (see nesle_render) */
};

enum { NESLE_DTYPE_U8 = 0, NESLE_DTYPE_I64 = 1, NESLE_DTYPE_F32 = 2, NESLE_DTYPE_U32 = 3, NESLE_DTYPE_U64 = 4 };

/* Size of the canonical full-state blob of one console ("NST1", little
 * endian; field offsets in nesle_amd/csrc/nes_layout.h). */
#define NESLE_STATE_BYTES 22896u

typedef struct nesle_batch nesle_batch;

typedef struct nesle_config {
    uint32_t num_envs;
    uint32_t frameskip;
    uint32_t max_instructions_per_frame; /* 0 selects 200,000 (cuda_module.cu:1467) */
    uint32_t reward_kind;                /* NESLE_REWARD_*                             */
    uint32_t x_lo, x_hi, done_addr, clip;
    float time_penalty;
    int32_t device;                      /* HIP device ordinal, -1 = current device    */
    uint32_t frames;                     /* 1 (default): keep the presentation snapshot
                                            that nesle_render draws; 0: RAM-only batch */
} nesle_config;

typedef struct nesle_view {
    void* data;         /* device pointer */
    int32_t ndim;
    int64_t shape[4];
    int32_t dtype;      /* NESLE_DTYPE_* */
    int32_t device_id;
} nesle_view;

typedef struct nesle_rom_info {
    uint32_t prg_rom_size;
    uint32_t chr_rom_size;
    uint32_t mapper;
    uint32_t submapper;
    uint32_t nametable_arrangement; /* 0 vertical, 1 horizontal, 2 four-screen */
    uint32_t has_trainer;
    uint32_t has_battery;
    uint32_t is_nes2;
} nesle_rom_info;

/* Defaults: SMB reward, frameskip 4, budget 200,000, current device, frames on. */
void nesle_config_init(nesle_config* cfg);

/* Largest batch: the step kernel addresses the interleaved RAM/PRG-RAM rows
 * (10,241 rows of round_up(num_envs, 256) bytes) with 32-bit offsets. */
#define NESLE_MAX_ENVS 262144u

/* Parse the iNES image, allocate device state, upload PRG/CHR and power every
 * console on.  Replaces CudaBatchBinding(num_envs, frameskip, rom_bytes):
 * cuda_module.cu:389-411 (+ allocate 978-1118, upload_rom 1209-1225,
 * reset_console 1227-1289).  num_envs must be 1..NESLE_MAX_ENVS. */
int nesle_create(const nesle_config* cfg, const uint8_t* ines, size_t ines_len, nesle_batch** out);

/* A batch without a cartridge: the reference's synthetic CudaBatch(num_envs,
 * frameskip) (cuda_module.cu:368-379, name "cuda").  No console runs; every
 * console's RAM holds the bytes the SMB reward rule reads (x position $006D/
 * $0086, y viewport $00B5, lives $075A, player state $000E, BCD time
 * $07F8-$07FA), powered on as cold_reset_synthetic_env does (batch_step.cuh:
 * 244-260).  nesle_step and nesle_synthetic_step (below) move it; reward_kind
 * is forced to the SMB rule, stats modes and snapshots are refused; frames
 * render blank (power-on PPU state).  Views, resets and the RAM observation
 * behave as for a console batch.  Fails like nesle_create for bad sizes. */
int nesle_create_synthetic(const nesle_config* cfg, nesle_batch** out);

/* One env-step of a synthetic batch.  apply_actions != 0 (the reference's
 * step(), apply_actions_kernel + step_reward_kernel, cuda_module.cu:319-354,
 * 546-565, kernels.cu:12-17): the pad moves x (Right +1, +1 more with B,
 * Left -1, clamped to 0..$FFFF) and every max(1, 24 / frameskip)-th step of
 * a console takes one from the BCD time, then the SMB rule scores it.
 * apply_actions == 0 (the reference's step_device(), which launches only the
 * reward kernel without a ROM, cuda_module.cu:620-633): the rule alone.
 * auto_reset: consoles done after the step power on again (rewards and
 * dones stay readable).  nesle_step on a synthetic batch is this call with
 * apply_actions = 1.  Fails with NESLE_EINVAL on a console batch. */
int nesle_synthetic_step(nesle_batch* b, int apply_actions, int auto_reset);

/* Install a snapshot bank (FCEUX FCS or canonical NST1 blobs, detected by
 * magic) and the per-env level map (host, num_envs bytes; null = all 0), then
 * reset every console from it.  Replaces the 4- and 5-argument constructors
 * (cuda_module.cu:413-467) and upload_snapshot_bank (1291-1415). */
int nesle_set_snapshots(nesle_batch* b, const uint8_t* const* blobs, const size_t* lens, uint32_t count,
                        const uint8_t* env_to_level);

/* Reference counting; the handle is freed when the count reaches zero.
 * Replaces ~CudaBatchBinding / release() (cuda_module.cu:423-425, 1120-1207)
 * and lets DLPack deleters outlive the Python object. */
void nesle_retain(nesle_batch* b);
void nesle_release(nesle_batch* b);

/* Reset every console (snapshot bank if installed, else power-on).
 * Replaces reset()/reset_device() (cuda_module.cu:469-531) minus the RGB copy. */
int nesle_reset(nesle_batch* b);

/* Masked reset; mask is num_envs bytes on host or device.  Replaces
 * reset_envs(mask) (cuda_module.cu:917-937).  With a device mask the call
 * only enqueues work on the batch's stream (no synchronisation). */
int nesle_reset_envs(nesle_batch* b, const uint8_t* mask, int mask_on_device);

/* Controller masks for the next step: num_envs uint8 masks or int64 values
 * already encoded as masks (low byte used), on host or device.  Replaces the
 * action copies of step()/step_device() (cuda_module.cu:540-544, 600-620). */
int nesle_set_actions(nesle_batch* b, const void* actions, int dtype, int on_device);

/* Run one env-step on every console (frameskip frames, reward/done, optional
 * fused auto-reset of done consoles), then refresh the RAM view.
 * stats_mode: 0 none, 1 per-console counters, 2 also opcode/PC histograms,
 * 3 per-console counters and the step kernel's census of the launch (how many
 * wave-iterations took each side path and the rare path, by cause, and the
 * shader cycles spent there; indices in nesle_amd/csrc/nes_layout.h,
 * namespace census; no reference counterpart).
 * Replaces launch_console_step_kernel (kernels.cu:145-158) and the
 * step_device/step_stats/step_profile sequences (cuda_module.cu:594-818). */
int nesle_step(nesle_batch* b, int auto_reset, int stats_mode);

/* Device view of one buffer (NESLE_VIEW_*, not OAM).  Replaces
 * ram_device/rewards_device/last_done_device (cuda_module.cu:854-902) and
 * frames_device (cuda_module.cu:871-886).  A frame view exists once
 * nesle_render has produced that output. */
int nesle_get_view(nesle_batch* b, int kind, nesle_view* out);

/* Synchronous copy of a view to host memory (bytes must equal its size).
 * Replaces ram()/oam() and the reward/done copies (cuda_module.cu:574-583,
 * 841-852, 904-915). */
int nesle_copy_to_host(nesle_batch* b, int kind, void* dst, size_t bytes);

/* Draw every console's frame from its presentation snapshot (frozen at the
 * last vblank; seeded from live state by full resets and state loads) into
 * the device buffers selected by `outputs` (NESLE_FRAME_*), allocated on
 * first use.  RGB and palette values follow the batched renderer
 * (batch_render.cuh:161-440, launched by render_device/launch_render_device,
 * cuda_module.cu:1435-1438, 865-869); GRAY84 is the 84x84 luma observation
 * of the reference's training wrappers (project/mario-rl-ram/src/mario_rl/
 * wrappers.py:209-215, Pillow BILINEAR).  With NESLE_FRAME_LIVE the frames
 * are drawn instead from every console's live state by the rules of the
 * reference CPU core's renderer (ppu.hpp:213-545, the frame its Console shows
 * and per-frame framebuffer hashes are taken of): current scroll, ctrl, mask,
 * OAM, palette and nametables, one scroll for the whole frame, a background
 * pixel opaque whenever its pattern colour is non-zero, CHR RAM read; the
 * presentation snapshot is left as it is.  Fails with NESLE_EINVAL on a
 * batch created with frames = 0.  Does not synchronise. */
int nesle_render(nesle_batch* b, uint32_t outputs);

/* Full state of one console as a canonical blob (host, NESLE_STATE_BYTES). */
int nesle_save_state(nesle_batch* b, uint32_t env, uint8_t* out_blob);

/* Load one canonical or FCS blob into the consoles selected by a host mask
 * (null = all).  Reward baselines are re-seeded from the loaded RAM. */
int nesle_load_state(nesle_batch* b, const uint8_t* blob, size_t len, const uint8_t* mask);

/* Copy console `env` into snapshot-bank slot `slot` (slots 0..count, the bank
 * grows by one when slot == count; at most 255 slots).  The capture the
 * reference only offers in its smoke tool (device_reset.cuh:72-259). */
int nesle_snapshot_capture(nesle_batch* b, uint32_t env, uint32_t slot);

/* Canonical blob of bank slot `slot` (host, NESLE_STATE_BYTES). */
int nesle_snapshot_export(nesle_batch* b, uint32_t slot, uint8_t* out_blob);

/* Replace the per-env level map (host, num_envs bytes, each < bank size). */
int nesle_set_env_levels(nesle_batch* b, const uint8_t* env_to_level);

/* Write one RAM byte in every console.  Replaces poke_ram (cuda_module.cu:939-946). */
int nesle_poke_ram(nesle_batch* b, uint32_t address, uint32_t value);

/* Write one RAM byte per console: values[env] (num_envs bytes, host or
 * device) into RAM[address & 0x7FF] of console env.  Reward baselines are
 * left as they are.  The per-console form of poke_ram (cuda_module.cu:939-946),
 * which writes one value into every console; no reference counterpart
 * otherwise.  Used to stagger episode counters across consoles.  With device
 * values the call only enqueues work on the batch's stream. */
int nesle_poke_ram_envs(nesle_batch* b, uint32_t address, const uint8_t* values, int on_device);

int nesle_synchronize(nesle_batch* b);
int nesle_set_stream(nesle_batch* b, void* hip_stream);

/* Step timing with HIP events recorded on the batch's stream while enabled
 * (enable resets the totals): before every step-kernel launch, between it
 * and the auto-reset's restore kernel, and after that.  nesle_get_timing
 * synchronises and returns the summed step-kernel milliseconds and the
 * number of timed steps; nesle_get_timing_split also returns the restore
 * kernel's milliseconds (0 for steps without auto-reset).  Any out pointer
 * may be null.  No reference counterpart: the reference measures kernels
 * only from its benchmark tools (cpp/tools/benchmark_cuda_kernels.cu:74-198). */
int nesle_set_timing(nesle_batch* b, int enable);
int nesle_get_timing(nesle_batch* b, double* total_ms, uint64_t* launches);
int nesle_get_timing_split(nesle_batch* b, double* step_ms, double* reset_ms, uint64_t* launches);

uint32_t nesle_num_envs(const nesle_batch* b);
uint32_t nesle_frameskip(const nesle_batch* b);
uint32_t nesle_num_levels(const nesle_batch* b);
int32_t nesle_device_id(const nesle_batch* b);

/* iNES header parse (rom.cpp:110-166). */
int nesle_parse_ines(const uint8_t* bytes, size_t len, nesle_rom_info* out);

/* FCEUX FCS save state -> canonical blob with the reference's warm-reset
 * field mapping (fcs.hpp:187-226, batch_step.cuh:174-242). */
int nesle_parse_fcs(const uint8_t* bytes, size_t len, uint8_t* out_blob);

const char* nesle_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* NESLE_HIP_H */
