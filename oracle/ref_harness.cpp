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

namespace {

constexpr std::size_t kStateBytes = 22896;

struct RefEnv {
    explicit RefEnv(nesle::RomImage rom) : console(std::move(rom)) { console.reset_cpu(cpu); }
    nesle::Console console;
    nesle::cpu::CpuState cpu;
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

}  // extern "C"
