// ref_harness.cpp -- C ABI over the reference's own CPU core, built from the
// reference sources where they lie (never copied into this repository).
//
// TEST INFRASTRUCTURE ONLY: compiled by oracle/Makefile into oracle/_ref/ and
// used to pin the oracle restatement (oracle/nes_oracle.cpp) and as the
// "reference" CPU baseline.  The product never links or loads it.
//
// It drives nesle::Console exactly as the reference's NativeConsole binding
// does (cpp/bindings/module.cpp:60-92): reset_cpu on construction, then per
// env-step controller1().set_buttons(mask) and `frameskip` x step_frame().
// The canonical state blob is the one documented in oracle/nes_oracle.cpp.
//
// Console/Ppu/StandardController keep their state private; a test harness
// needs all of it for the full-state hash, so access specifiers are widened
// for this translation unit only (standard headers are included first so the
// redefinition cannot reach them).
#include <algorithm>
#include <array>
#include <atomic>
#include <chrono>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <memory>
#include <span>
#include <stdexcept>
#include <string>
#include <string_view>
#include <thread>
#include <utility>
#include <vector>

#define private public
#include "nesle/console.hpp"
#include "nesle/rom.hpp"
#undef private
// The batched core's PPU timing and renderer, compiled as host C++ (the
// reference's own host tests do the same, tests/cpp/test_cuda_render.cpp).
#include "nesle/cuda/batch_ppu.cuh"
#include "nesle/cuda/batch_render.cuh"

namespace {

constexpr std::size_t kStateBytes = 22896;

// The batched core's presentation state of one console, advanced beside the
// CPU core by batch_ppu_step_env_hot (batch_ppu.cuh:183-269) with the
// console's registers and video memory after each instruction: the frame-start
// latch (lat_*) and the vblank snapshot (snap_*).
struct Shadow {
    std::uint8_t lat_sx = 0, lat_sy = 0, lat_ctrl = 0;
    std::uint8_t sx_start = 0, sy_start = 0, ctrl_start = 0, sx_end = 0, sy_end = 0, ctrl_end = 0, mask = 0;
    std::array<std::uint8_t, 256> oam{};
    std::array<std::uint8_t, 2048> nt{};
    std::array<std::uint8_t, 32> palette{};
};

struct RefEnv {
    explicit RefEnv(nesle::RomImage rom) : console(std::move(rom)) { console.reset_cpu(cpu); }
    nesle::Console console;
    nesle::cpu::CpuState cpu;
    Shadow shadow;
};

thread_local std::string g_error;

void put16(std::uint8_t* o, std::size_t off, std::uint16_t v) { o[off] = v & 0xFF; o[off + 1] = v >> 8; }
void put32(std::uint8_t* o, std::size_t off, std::uint32_t v) { for (int i = 0; i < 4; ++i) o[off + i] = (v >> (8 * i)) & 0xFF; }
void put64(std::uint8_t* o, std::size_t off, std::uint64_t v) { for (int i = 0; i < 8; ++i) o[off + i] = (v >> (8 * i)) & 0xFF; }

std::uint64_t splitmix64(std::uint64_t x) {
    std::uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

}  // namespace

extern "C" {

const char* ref_last_error() { return g_error.c_str(); }

void* ref_create(const std::uint8_t* ines, std::size_t len) {
    try {
        auto rom = nesle::parse_ines(std::span<const std::uint8_t>(ines, len));
        return new RefEnv(std::move(rom));
    } catch (const std::exception& ex) {
        g_error = ex.what();
        return nullptr;
    }
}

void ref_destroy(void* h) { delete static_cast<RefEnv*>(h); }

// The reference CPU core's frame (ppu.hpp:213-230): 240 x 256 x RGB.
void ref_render_rgb(void* h, std::uint8_t* out) {
    const auto frame = static_cast<RefEnv*>(h)->console.ppu().render_rgb_frame();
    std::memcpy(out, frame.data(), frame.size());
}

std::int64_t ref_step(void* h, std::uint8_t buttons, std::uint32_t frameskip, std::uint64_t max_instructions) {
    auto* e = static_cast<RefEnv*>(h);
    try {
        e->console.controller1().set_buttons(buttons);
        std::uint64_t n = 0;
        for (std::uint32_t f = 0; f < frameskip; ++f) n += e->console.step_frame(e->cpu, max_instructions).instructions;
        return static_cast<std::int64_t>(n);
    } catch (const std::exception& ex) {
        g_error = ex.what();
        return -1;
    }
}

void ref_save(void* h, std::uint8_t* o) {
    const auto* e = static_cast<RefEnv*>(h);
    const auto& c = e->console;
    const auto& p = c.ppu_;
    std::memset(o, 0, kStateBytes);
    std::memcpy(o, "NST1", 4);
    put16(o, 4, e->cpu.pc);
    o[6] = e->cpu.a; o[7] = e->cpu.x; o[8] = e->cpu.y; o[9] = e->cpu.sp; o[10] = e->cpu.p;
    o[11] = p.nmi_pending_ ? 1 : 0;
    put64(o, 12, e->cpu.cycles);
    put64(o, 20, p.frame_);
    put32(o, 28, static_cast<std::uint32_t>(p.scanline_) * 341u + p.dot_);
    o[32] = p.ctrl_; o[33] = p.mask_; o[34] = p.status_; o[35] = p.oam_addr_;
    o[36] = p.open_bus_; o[37] = p.read_buffer_;
    put16(o, 38, p.v_); put16(o, 40, p.t_);
    o[42] = p.x_; o[43] = p.w_ ? 1 : 0; o[44] = p.scroll_x_; o[45] = p.scroll_y_;
    o[46] = c.controller1_.buttons_; o[47] = c.controller1_.shift_register_;
    o[48] = c.controller1_.shift_count_; o[49] = c.controller1_.strobe_ ? 1 : 0;
    o[50] = c.controller2_.shift_count_;
    o[51] = 0;
    put32(o, 52, c.pending_dma_cycles_);
    std::memcpy(o + 56, c.apu_io_.data(), 24);
    std::memcpy(o + 80, c.cpu_ram_.data(), 2048);
    std::memcpy(o + 2128, c.prg_ram_.data(), 8192);
    std::memcpy(o + 10320, p.oam_.data(), 256);
    std::memcpy(o + 10576, p.palette_ram_.data(), 32);
    std::memcpy(o + 10608, p.nametable_ram_.data(), 4096);
    std::memcpy(o + 14704, p.chr_ram_.data(), 8192);
}

// Inverse of ref_save: every field of the canonical blob into the Console.
// Pad 2 has no buttons; it shares pad 1's strobe line.
void ref_load(void* h, const std::uint8_t* s) {
    auto* e = static_cast<RefEnv*>(h);
    auto& c = e->console;
    auto& p = c.ppu_;
    auto u16 = [&](std::size_t off) { return static_cast<std::uint16_t>(s[off] | (s[off + 1] << 8)); };
    auto u32 = [&](std::size_t off) {
        std::uint32_t r = 0;
        for (int i = 0; i < 4; ++i) r |= std::uint32_t(s[off + i]) << (8 * i);
        return r;
    };
    auto u64 = [&](std::size_t off) {
        std::uint64_t r = 0;
        for (int i = 0; i < 8; ++i) r |= std::uint64_t(s[off + i]) << (8 * i);
        return r;
    };
    e->cpu.pc = u16(4);
    e->cpu.a = s[6]; e->cpu.x = s[7]; e->cpu.y = s[8]; e->cpu.sp = s[9]; e->cpu.p = s[10];
    p.nmi_pending_ = s[11] != 0;
    e->cpu.cycles = u64(12);
    p.frame_ = u64(20);
    const std::uint32_t fd = u32(28);
    p.scanline_ = static_cast<std::int16_t>(fd / 341u);
    p.dot_ = static_cast<std::uint16_t>(fd % 341u);
    p.ctrl_ = s[32]; p.mask_ = s[33]; p.status_ = s[34]; p.oam_addr_ = s[35];
    p.open_bus_ = s[36]; p.read_buffer_ = s[37];
    p.v_ = u16(38); p.t_ = u16(40);
    p.x_ = s[42]; p.w_ = s[43] != 0; p.scroll_x_ = s[44]; p.scroll_y_ = s[45];
    c.controller1_.buttons_ = s[46]; c.controller1_.shift_register_ = s[47];
    c.controller1_.shift_count_ = s[48]; c.controller1_.strobe_ = s[49] != 0;
    c.controller2_.buttons_ = 0; c.controller2_.shift_register_ = 0;
    c.controller2_.shift_count_ = s[50]; c.controller2_.strobe_ = s[49] != 0;
    c.pending_dma_cycles_ = u32(52);
    std::memcpy(c.apu_io_.data(), s + 56, 24);
    std::memcpy(c.cpu_ram_.data(), s + 80, 2048);
    std::memcpy(c.prg_ram_.data(), s + 2128, 8192);
    std::memcpy(p.oam_.data(), s + 10320, 256);
    std::memcpy(p.palette_ram_.data(), s + 10576, 32);
    std::memcpy(p.nametable_ram_.data(), s + 10608, 4096);
    std::memcpy(p.chr_ram_.data(), s + 14704, 8192);
}

// Console::step_cpu_instruction (console.hpp:108-135); returns CPU cycles
// (NMI and DMA included), frames completed in *frames, -1 on an exception.
std::int64_t ref_step_instruction(void* h, std::uint32_t* frames) {
    auto* e = static_cast<RefEnv*>(h);
    try {
        const auto r = e->console.step_cpu_instruction(e->cpu);
        if (frames) *frames = r.frames_completed;
        return static_cast<std::int64_t>(r.cpu_cycles);
    } catch (const std::exception& ex) {
        g_error = ex.what();
        return -1;
    }
}

// Same contract as oracle_run_batch (oracle/nes_oracle.cpp), over the
// reference Console.  Used as the "reference" CPU baseline.
double ref_run_batch(const std::uint8_t* ines, std::size_t len, std::uint32_t n_envs,
                     std::uint32_t steps, std::uint32_t frameskip, std::uint64_t seed,
                     std::uint32_t threads, std::uint64_t* checksum, std::uint64_t* instructions) {
    nesle::RomImage rom;
    try {
        rom = nesle::parse_ines(std::span<const std::uint8_t>(ines, len));
    } catch (const std::exception& ex) {
        g_error = ex.what();
        return -1.0;
    }
    threads = std::max(1u, std::min(threads, n_envs));
    std::atomic<std::uint64_t> sum{0}, instr{0};
    std::atomic<bool> failed{false};
    const auto t0 = std::chrono::steady_clock::now();
    std::vector<std::thread> pool;
    for (std::uint32_t t = 0; t < threads; ++t) {
        pool.emplace_back([&, t]() {
            const auto lo = static_cast<std::uint32_t>(std::uint64_t(n_envs) * t / threads);
            const auto hi = static_cast<std::uint32_t>(std::uint64_t(n_envs) * (t + 1) / threads);
            std::uint64_t local = 0, li = 0;
            try {
                for (std::uint32_t env = lo; env < hi; ++env) {
                    auto e = std::make_unique<RefEnv>(rom);
                    for (std::uint32_t k = 0; k < steps; ++k) {
                        e->console.controller1().set_buttons(
                            static_cast<std::uint8_t>(splitmix64(seed ^ (std::uint64_t(env) << 32) ^ k) & 0xFF));
                        for (std::uint32_t f = 0; f < frameskip; ++f)
                            li += e->console.step_frame(e->cpu, 200000).instructions;
                    }
                    std::uint64_t h = 0xCBF29CE484222325ull;
                    for (auto b : e->console.cpu_ram_) { h ^= b; h *= 0x100000001B3ull; }
                    local ^= h;
                }
            } catch (...) {
                failed = true;
            }
            sum ^= local;
            instr += li;
        });
    }
    for (auto& th : pool) th.join();
    const double secs = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    if (failed) {
        g_error = "exception during reference batch run";
        return -1.0;
    }
    if (checksum) *checksum = sum.load();
    if (instructions) *instructions = instr.load();
    return secs;
}

// Same contract as oracle_run_levels (oracle/nes_oracle.cpp), over the
// reference Console: start from snapshot blobs with a per-console done byte,
// re-load the console's blob after an env-step that leaves the byte at 0.
double ref_run_levels(const std::uint8_t* ines, std::size_t len, const std::uint8_t* blobs, std::uint32_t n_levels,
                      const std::uint8_t* levels, const std::uint8_t* done_init, std::uint32_t done_addr,
                      std::uint32_t n_envs, std::uint32_t steps, std::uint32_t frameskip, std::uint64_t seed,
                      std::uint64_t step0, std::uint32_t threads, std::uint64_t* checksum,
                      std::uint64_t* instructions, std::uint64_t* resets) {
    nesle::RomImage rom;
    try {
        rom = nesle::parse_ines(std::span<const std::uint8_t>(ines, len));
    } catch (const std::exception& ex) {
        g_error = ex.what();
        return -1.0;
    }
    for (std::uint32_t e = 0; e < n_envs; ++e)
        if (levels[e] >= n_levels) {
            g_error = "level out of range";
            return -1.0;
        }
    threads = std::max(1u, std::min(threads, n_envs));
    done_addr &= 0x7FF;
    std::atomic<std::uint64_t> sum{0}, instr{0}, rs{0};
    std::atomic<bool> failed{false};
    const auto t0 = std::chrono::steady_clock::now();
    std::vector<std::thread> pool;
    for (std::uint32_t t = 0; t < threads; ++t) {
        pool.emplace_back([&, t]() {
            const auto lo = static_cast<std::uint32_t>(std::uint64_t(n_envs) * t / threads);
            const auto hi = static_cast<std::uint32_t>(std::uint64_t(n_envs) * (t + 1) / threads);
            std::uint64_t local = 0, li = 0, lr = 0;
            try {
                for (std::uint32_t env = lo; env < hi; ++env) {
                    const std::uint8_t* b = blobs + static_cast<std::size_t>(levels[env]) * kStateBytes;
                    auto e = std::make_unique<RefEnv>(rom);
                    ref_load(e.get(), b);
                    e->console.cpu_ram_[done_addr] = done_init[env];
                    for (std::uint32_t k = 0; k < steps; ++k) {
                        e->console.controller1().set_buttons(static_cast<std::uint8_t>(
                            splitmix64(seed ^ (std::uint64_t(env) << 32) ^ (step0 + k)) & 0xFF));
                        for (std::uint32_t f = 0; f < frameskip; ++f)
                            li += e->console.step_frame(e->cpu, 200000).instructions;
                        if (e->console.cpu_ram_[done_addr] == 0) {
                            ref_load(e.get(), b);
                            ++lr;
                        }
                    }
                    std::uint64_t h = 0xCBF29CE484222325ull;
                    for (auto v : e->console.cpu_ram_) { h ^= v; h *= 0x100000001B3ull; }
                    local ^= h;
                }
            } catch (...) {
                failed = true;
            }
            sum ^= local;
            instr += li;
            rs += lr;
        });
    }
    for (auto& th : pool) th.join();
    const double secs = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    if (failed) {
        g_error = "exception during reference batch run";
        return -1.0;
    }
    if (checksum) *checksum = sum.load();
    if (instructions) *instructions = instr.load();
    if (resets) *resets = rs.load();
    return secs;
}


// ---- the batched core's frame path (batch_ppu.cuh, batch_render.cuh) ----------

// Presentation state seeded from live state, as a full reset of the batched
// core does (cuda_module.cu:1440-1463).
void ref_present_seed(void* h) {
    auto* e = static_cast<RefEnv*>(h);
    const auto& p = e->console.ppu_;
    auto& sh = e->shadow;
    sh.lat_sx = sh.sx_start = sh.sx_end = p.scroll_x_;
    sh.lat_sy = sh.sy_start = sh.sy_end = p.scroll_y_;
    sh.lat_ctrl = sh.ctrl_start = sh.ctrl_end = p.ctrl_;
    sh.mask = p.mask_;
    std::memcpy(sh.oam.data(), p.oam_.data(), 256);
    std::memcpy(sh.nt.data(), p.nametable_ram_.data(), 2048);
    std::memcpy(sh.palette.data(), p.palette_ram_.data(), 32);
}

// One env-step of the CPU core (Console::step_frame, console.hpp:137-150,
// `frameskip` times) in which every instruction's PPU dots also advance the
// batched core's timing (batch_ppu_step_env_hot) over a one-console
// BatchBuffers that points at the console's registers and video memory as the
// instruction left them -- the batched core's order: the instruction's
// register writes, then its dots.  Returns instructions, -1 on an exception.
std::int64_t ref_present_step(void* h, std::uint8_t buttons, std::uint32_t frameskip, std::uint64_t max_instructions) {
    auto* e = static_cast<RefEnv*>(h);
    auto& c = e->console;
    auto& p = c.ppu_;
    auto& sh = e->shadow;
    std::uint8_t ctrl = 0, mask = 0, status = 0, oam_addr = 0, nmi = 0, sx = 0, sy = 0;
    std::uint32_t frame_dot = static_cast<std::uint32_t>(p.scanline_) * 341u + p.dot_;
    std::uint64_t frame_count = p.frame_;
    nesle::cuda::BatchBuffers b{};
    b.ppu.ctrl = &ctrl;
    b.ppu.mask = &mask;
    b.ppu.status = &status;
    b.ppu.oam_addr = &oam_addr;
    b.ppu.nmi_pending = &nmi;
    b.ppu.frame_dot = &frame_dot;
    b.ppu.frame = &frame_count;
    b.ppu.scroll_x = &sx;
    b.ppu.scroll_y = &sy;
    b.ppu.oam = p.oam_.data();
    b.ppu.nametable_ram = p.nametable_ram_.data();
    b.ppu.palette_ram = p.palette_ram_.data();
    b.ppu.lat_scroll_x = &sh.lat_sx;
    b.ppu.lat_scroll_y = &sh.lat_sy;
    b.ppu.lat_ctrl = &sh.lat_ctrl;
    b.ppu.snap_scroll_x_start = &sh.sx_start;
    b.ppu.snap_scroll_y_start = &sh.sy_start;
    b.ppu.snap_ctrl_start = &sh.ctrl_start;
    b.ppu.snap_scroll_x_end = &sh.sx_end;
    b.ppu.snap_scroll_y_end = &sh.sy_end;
    b.ppu.snap_ctrl_end = &sh.ctrl_end;
    b.ppu.snap_mask = &sh.mask;
    b.ppu.snap_oam = sh.oam.data();
    b.ppu.snap_nametable = sh.nt.data();
    b.ppu.snap_palette = sh.palette.data();
    try {
        c.controller1().set_buttons(buttons);
        std::int64_t n = 0;
        for (std::uint32_t f = 0; f < frameskip; ++f) {
            for (std::uint64_t i = 0; i < max_instructions; ++i) {
                const auto r = c.step_cpu_instruction(e->cpu);
                ++n;
                nesle::cuda::PpuHotState hot;
                hot.frame_dot = frame_dot;
                hot.frame = frame_count;
                hot.ctrl = p.ctrl_;
                hot.mask = p.mask_;
                sx = p.scroll_x_;
                sy = p.scroll_y_;
                nesle::cuda::batch_ppu_step_env_hot(b, 0, r.ppu_cycles, hot);
                frame_dot = hot.frame_dot;
                frame_count = hot.frame;
                if (r.frames_completed != 0) break;
            }
        }
        return n;
    } catch (const std::exception& ex) {
        g_error = ex.what();
        return -1;
    }
}

// The shadow presentation state: [0..6] frame-start x, y, ctrl, frame-end
// x, y, ctrl, mask; [7..9] the latch x, y, ctrl; [16..271] OAM; [272..303]
// palette; [304..2351] nametable RAM.
void ref_present_get(void* h, std::uint8_t* out) {
    const auto& sh = static_cast<RefEnv*>(h)->shadow;
    const std::uint8_t head[10] = {sh.sx_start, sh.sy_start, sh.ctrl_start, sh.sx_end, sh.sy_end,
                                   sh.ctrl_end, sh.mask, sh.lat_sx, sh.lat_sy, sh.lat_ctrl};
    std::memset(out, 0, 16);
    std::memcpy(out, head, 10);
    std::memcpy(out + 16, sh.oam.data(), 256);
    std::memcpy(out + 272, sh.palette.data(), 32);
    std::memcpy(out + 304, sh.nt.data(), 2048);
}

// One frame of the batched core's renderer (batch_render.cuh:161-440) for
// one console whose state is given directly: CHR ROM (chr_size 0 = CHR RAM,
// which that renderer reads as 0), the nametable arrangement (0 vertical,
// 1 horizontal, 2 four-screen), f = frame-start x, y, ctrl, frame-end x, y,
// ctrl, mask, and OAM (256), nametable RAM (4,096 bytes: four-screen reads
// all of it) and palette RAM (32).  mode bit 0: from a presentation snapshot
// holding these (render_batch_rgb_frame_env through
// resolve_render_env_views), else from live state with the frame-end
// scroll/ctrl and no snapshot; bit 1: the per-pixel renderer
// (render_batch_rgb_pixel_env, what the reference's device kernel runs)
// instead of the serial frame renderer.  out: 240 x 256 x RGB.
void ref_batch_render(const std::uint8_t* chr, std::uint32_t chr_size, std::uint32_t arrangement,
                      const std::uint8_t* f, const std::uint8_t* oam, const std::uint8_t* nt,
                      const std::uint8_t* palette, std::uint32_t mode, std::uint8_t* out) {
    std::vector<std::uint8_t> chr_copy(chr, chr + chr_size);
    std::array<std::uint8_t, 256> oam_copy{};
    std::array<std::uint8_t, 4096> nt_copy{};
    std::array<std::uint8_t, 32> pal_copy{};
    std::memcpy(oam_copy.data(), oam, 256);
    std::memcpy(nt_copy.data(), nt, 4096);
    std::memcpy(pal_copy.data(), palette, 32);
    std::uint8_t sx_start = f[0], sy_start = f[1], ctrl_start = f[2], sx_end = f[3], sy_end = f[4], ctrl_end = f[5];
    std::uint8_t mask = f[6];
    std::uint8_t live_ctrl = ctrl_end, live_mask = mask, live_sx = sx_end, live_sy = sy_end;
    nesle::cuda::BatchBuffers b{};
    b.cart.chr_rom = chr_size != 0 ? chr_copy.data() : nullptr;
    b.cart.chr_rom_size = chr_size;
    b.cart.nametable_arrangement = static_cast<std::uint8_t>(arrangement);
    b.ppu.ctrl = &live_ctrl;
    b.ppu.mask = &live_mask;
    b.ppu.scroll_x = &live_sx;
    b.ppu.scroll_y = &live_sy;
    b.ppu.oam = oam_copy.data();
    b.ppu.nametable_ram = nt_copy.data();
    b.ppu.palette_ram = pal_copy.data();
    if (mode & 1) {
        b.ppu.snap_scroll_x_start = &sx_start;
        b.ppu.snap_scroll_y_start = &sy_start;
        b.ppu.snap_ctrl_start = &ctrl_start;
        b.ppu.snap_scroll_x_end = &sx_end;
        b.ppu.snap_scroll_y_end = &sy_end;
        b.ppu.snap_ctrl_end = &ctrl_end;
        b.ppu.snap_mask = &mask;
        b.ppu.snap_oam = oam_copy.data();
        b.ppu.snap_nametable = nt_copy.data();
        b.ppu.snap_palette = pal_copy.data();
    }
    b.frames_rgb = out;
    if (mode & 2) {
        auto views = nesle::cuda::resolve_render_env_views(b, 0);
        for (std::uint32_t px = 0; px < 240u * 256u; ++px)
            nesle::cuda::render_batch_rgb_pixel_env(b, views.hud, views.play, 0, views.split_y, px);
    } else {
        nesle::cuda::render_batch_rgb_frame_env(b, 0);
    }
}

}  // extern "C"
