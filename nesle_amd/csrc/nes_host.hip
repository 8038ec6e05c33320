// nes_host.hip -- host side of libnesle_hip.so: the C ABI declared in
// include/nesle_hip.h.  Owns every device buffer of a batch (one arena
// allocation), parses cartridges and snapshots, and sequences the kernels of
// nes_kernels.hip on the batch's stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstring>
#include <exception>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "../../include/nesle_hip.h"
#include "nes_launch.h"
#include "nes_layout.h"
#include "nes_render.h"

using nesle::DeviceState;
namespace blob = nesle::blob;

namespace {

thread_local std::string g_error;

struct InvalidArgument : std::invalid_argument {
    using std::invalid_argument::invalid_argument;
};
struct DeviceError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw DeviceError(std::string(what) + ": " + hipGetErrorString(e));
}

template <typename F>
int guarded(F&& fn) {
    try {
        fn();
        return NESLE_OK;
    } catch (const InvalidArgument& ex) {
        g_error = ex.what();
        return NESLE_EINVAL;
    } catch (const std::invalid_argument& ex) {
        g_error = ex.what();
        return NESLE_EINVAL;
    } catch (const DeviceError& ex) {
        g_error = ex.what();
        return NESLE_EDEVICE;
    } catch (const std::exception& ex) {
        g_error = ex.what();
        return NESLE_ERUNTIME;
    } catch (...) {
        g_error = "unknown error";
        return NESLE_ERUNTIME;
    }
}

// ---- iNES (the reference's rom.cpp:110-166 rules) ------------------------------
struct Rom {
    nesle_rom_info info{};
    std::vector<std::uint8_t> prg, chr;
};

Rom parse_ines(const std::uint8_t* b, std::size_t n) {
    if (b == nullptr || n < 16) throw InvalidArgument("iNES image shorter than its 16-byte header");
    if (b[0] != 'N' || b[1] != 'E' || b[2] != 'S' || b[3] != 0x1A)
        throw InvalidArgument("iNES image: bad magic, the first four bytes are not N E S 0x1A");
    Rom r;
    const bool nes2 = (b[7] & 0x0C) == 0x08;
    if (nes2 && b[9] != 0) throw InvalidArgument("NES 2.0 image with extended (exponent form) PRG/CHR sizes: not handled");
    r.info.is_nes2 = nes2;
    r.info.mapper = (b[6] >> 4) | (b[7] & 0xF0);
    if (nes2) {
        r.info.mapper |= static_cast<std::uint32_t>(b[8] & 0x0F) << 8;
        r.info.submapper = b[8] >> 4;
    }
    r.info.has_trainer = (b[6] & 0x04) != 0;
    r.info.has_battery = (b[6] & 0x02) != 0;
    r.info.nametable_arrangement = (b[6] & 0x08) ? 2u : ((b[6] & 0x01) ? 0u : 1u);
    r.info.prg_rom_size = b[4] * 16384u;
    r.info.chr_rom_size = b[5] * 8192u;
    std::size_t off = 16 + (r.info.has_trainer ? 512 : 0);
    if (n < off + r.info.prg_rom_size + r.info.chr_rom_size)
        throw InvalidArgument("iNES image truncated: fewer bytes than its header declares for trainer, PRG and CHR");
    r.prg.assign(b + off, b + off + r.info.prg_rom_size);
    off += r.info.prg_rom_size;
    r.chr.assign(b + off, b + off + r.info.chr_rom_size);
    return r;
}

// ---- FCEUX FCS -> canonical blob (fcs.hpp:187-226 + the warm-reset mapping of
//      batch_step.cuh:174-242: frame position, NMI, pads, DMA and scroll start
//      at zero) ----------------------------------------------------------------------
std::uint32_t rd_le32(const std::uint8_t* p) {
    return p[0] | (p[1] << 8) | (p[2] << 16) | (static_cast<std::uint32_t>(p[3]) << 24);
}

void fcs_to_blob(const std::uint8_t* d, std::size_t n, std::uint8_t* o) {
    if (n < 16) throw std::runtime_error("FCEUX state: fewer than 16 bytes, no room for the file header");
    if (d[0] != 'F' || d[1] != 'C' || d[2] != 'S' || d[3] != 0xFF)
        throw std::runtime_error("FCEUX state: the file does not start with the signature F C S 0xFF");
    std::memset(o, 0, blob::kBytes);
    std::memcpy(o, "NST1", 4);
    o[blob::kSp] = 0xFD;
    o[blob::kP] = 0x24;
    o[blob::kC1Count] = 8;
    o[blob::kC2Count] = 8;
    auto walk = [&](const std::uint8_t* pay, std::size_t len, int tag) {
        std::size_t off = 0;
        while (off + 8 <= len) {
            std::size_t nl = 4;
            while (nl > 0 && pay[off + nl - 1] == 0) --nl;
            const std::string name(reinterpret_cast<const char*>(pay + off), nl);
            const std::uint32_t size = rd_le32(pay + off + 4);
            off += 8;
            if (off + size > len) throw std::runtime_error("FCEUX state: field " + name + " of a section runs beyond that section");
            const std::uint8_t* v = pay + off;
            auto fixed = [&](std::uint32_t dst, std::uint32_t want, const char* label) {
                if (size != want)
                    throw std::runtime_error(std::string("FCEUX state: field ") + label + " holds " + std::to_string(size) +
                                             " bytes where " + std::to_string(want) + " belong");
                std::memcpy(o + dst, v, want);
            };
            if (tag == 1) {
                if (name == "PC") {
                    if (size != 2) throw std::runtime_error("FCEUX state: field CPU.PC holds other than 2 bytes");
                    o[blob::kPc] = v[0];
                    o[blob::kPc + 1] = v[1];
                } else if (size == 1 && (name == "A" || name == "X" || name == "Y" || name == "S" || name == "P")) {
                    const std::uint32_t at = name == "A" ? blob::kA : name == "X" ? blob::kX : name == "Y" ? blob::kY
                                           : name == "S" ? blob::kSp : blob::kP;
                    o[at] = v[0];
                } else if (name == "RAM") {
                    fixed(blob::kRam, nesle::kRamBytes, "CPU.RAM");
                }
            } else if (tag == 3) {
                if (name == "NTAR") {
                    fixed(blob::kNametable, 2048, "PPU.NTAR");
                } else if (name == "PRAM") {
                    fixed(blob::kPalette, nesle::kPaletteBytes, "PPU.PRAM");
                } else if (name == "SPRA") {
                    fixed(blob::kOam, nesle::kOamBytes, "PPU.SPRA");
                } else if (name == "PPUR") {
                    if (size < 3) throw std::runtime_error("FCEUX state: field PPU.PPUR holds fewer than 3 bytes");
                    o[blob::kCtrl] = v[0];
                    o[blob::kMask] = v[1];
                    o[blob::kStatus] = v[2];
                } else if (name == "PSPL" && size == 1) {
                    o[blob::kOamAddr] = v[0];
                } else if (name == "XOFF" && size == 1) {
                    o[blob::kFineX] = v[0] & 7;
                } else if (name == "VTGL" && size == 1) {
                    o[blob::kW] = v[0] & 1;
                } else if (name == "RADD" && size == 2) {
                    o[blob::kV] = v[0];
                    o[blob::kV + 1] = v[1];
                } else if (name == "TADD" && size == 2) {
                    o[blob::kT] = v[0];
                    o[blob::kT + 1] = v[1];
                } else if (name == "VBUF" && size == 1) {
                    o[blob::kReadBuffer] = v[0];
                } else if (name == "PGEN" && size == 1) {
                    o[blob::kOpenBus] = v[0];
                }
            } else if (tag == 16) {
                if (name == "WRAM") fixed(blob::kPrgRam, nesle::kPrgRamBytes, "CART.WRAM");
            }
            off += size;
        }
        if (off != len) throw std::runtime_error("FCEUX state: a section ends with a partial field header");
    };
    std::size_t off = 16;
    while (off + 5 <= n) {
        const int tag = d[off];
        const std::uint32_t size = rd_le32(d + off + 1);
        off += 5;
        if (off + size > n) throw std::runtime_error("FCEUX state: a section runs beyond the end of the file");
        if (tag == 1 || tag == 3 || tag == 16) walk(d + off, size, tag);
        off += size;
    }
    if (off != n) throw std::runtime_error("FCEUX state: the file ends with a partial section header");
}

// A snapshot blob in either format, as a canonical blob.
std::vector<std::uint8_t> to_canonical(const std::uint8_t* d, std::size_t n) {
    std::vector<std::uint8_t> out(blob::kBytes);
    if (n >= 4 && std::memcmp(d, "NST1", 4) == 0) {
        if (n != blob::kBytes) throw InvalidArgument("NST1 state blob must be " + std::to_string(blob::kBytes) + " bytes");
        std::memcpy(out.data(), d, n);
    } else {
        fcs_to_blob(d, n, out.data());
    }
    return out;
}

std::size_t align_up(std::size_t v, std::size_t a) { return (v + a - 1) / a * a; }

}  // namespace

struct nesle_batch {
    std::atomic<int> refs{1};
    // The ROM-less synthetic batch (nesle_create_synthetic): no console runs;
    // steps and resets are the synthetic kernels over RAM and the reward.
    bool synthetic = false;
    std::uint32_t* d_step_counts = nullptr;   // synthetic: env-steps per console
    int device = 0;
    hipStream_t stream = nullptr;
    nesle_config cfg{};
    Rom rom;
    std::uint32_t pitch = 0;
    void* arena = nullptr;
    DeviceState ds{};
    std::uint8_t* d_prg = nullptr;
    std::uint8_t* d_chr = nullptr;
    std::uint8_t* d_obs = nullptr;     // [n][2048] RAM observation
    std::uint8_t* d_mask = nullptr;    // [n] scratch mask
    std::uint8_t* d_blob = nullptr;    // one canonical blob of staging
    std::uint8_t* d_levels = nullptr;  // [n] env_to_level
    std::uint8_t* d_bank = nullptr;    // num_levels blobs
    std::uint32_t num_levels = 0;
    std::uint32_t bank_capacity = 0;
    void* stats_arena = nullptr;
    // Frames: render outputs (allocated on first use) and the resample tables.
    std::uint8_t* d_frame_rgb = nullptr;
    std::uint8_t* d_frame_palette = nullptr;
    std::uint8_t* d_gray84 = nullptr;
    std::uint8_t* d_live_records = nullptr;   // records of live state (NESLE_FRAME_LIVE renders)
    void* d_render_tables = nullptr;   // render::Tables
    // Step timing: three events per step (before the step kernel, between it
    // and the auto-reset's restore kernel, after that), folded into the
    // totals once the last has completed.
    struct Marks { hipEvent_t start, stepped, reset; bool restored; };
    bool timing = false;
    std::vector<Marks> events;  // recorded, not yet folded
    std::vector<Marks> spare;
    double timed_ms = 0.0;        // step kernel
    double timed_reset_ms = 0.0;  // restore kernel of the auto-reset
    std::uint64_t timed_launches = 0;

    ~nesle_batch() {
        if (device >= 0) (void)hipSetDevice(device);
        for (auto* list : {&events, &spare})
            for (auto& e : *list) {
                (void)hipEventDestroy(e.start);
                (void)hipEventDestroy(e.stepped);
                (void)hipEventDestroy(e.reset);
            }
        (void)hipFree(arena);
        (void)hipFree(d_bank);
        (void)hipFree(stats_arena);
        (void)hipFree(d_frame_rgb);
        (void)hipFree(d_frame_palette);
        (void)hipFree(d_gray84);
        (void)hipFree(d_live_records);
        (void)hipFree(d_step_counts);
        (void)hipFree(d_render_tables);
    }

    void activate() const { hip_check(hipSetDevice(device), "hipSetDevice"); }

    void sync() const { hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize"); }

    std::uint32_t n() const { return cfg.num_envs; }

    void allocate() {
        const std::size_t n = cfg.num_envs, P = pitch;
        struct Slot { void** dst; std::size_t bytes; };
        std::vector<Slot> slots;
        auto add = [&](auto** p, std::size_t bytes) { slots.push_back({reinterpret_cast<void**>(p), bytes}); };
        add(&d_prg, nesle::kPrgRomMax);
        add(&d_chr, std::max<std::size_t>(rom.chr.size(), 16));
        add(&ds.pc, 2 * n); add(&ds.a, n); add(&ds.x, n); add(&ds.y, n); add(&ds.sp, n); add(&ds.p, n);
        add(&ds.fault, n); add(&ds.cycles, 8 * n);
        add(&ds.frame_dot, 4 * n); add(&ds.frame, 8 * n); add(&ds.ctrl, n); add(&ds.mask, n); add(&ds.status, n);
        add(&ds.nmi_pending, n); add(&ds.oam_addr, n); add(&ds.open_bus, n); add(&ds.read_buffer, n);
        add(&ds.v, 2 * n); add(&ds.t, 2 * n); add(&ds.fine_x, n); add(&ds.w, n); add(&ds.scroll_x, n);
        add(&ds.scroll_y, n); add(&ds.c1_buttons, n); add(&ds.c1_shift, n); add(&ds.c1_count, n);
        add(&ds.strobe, n); add(&ds.c2_count, n);
        add(&ds.apu_io, nesle::kApuIoBytes * P);
        // RAM rows 0-2047 and PRG RAM rows 2048-10239 form one interleaved array,
        // so the step kernel reaches both with one row * pitch + env offset.
        // Plus one spare row that the step kernel's lanes with nothing to store write to.
        add(&ds.ram, static_cast<std::size_t>(nesle::kRamBytes + nesle::kPrgRamBytes + 1) * P);
        add(&ds.vram, static_cast<std::size_t>(ds.vram_stride) * n);
        if (rom.chr.empty()) add(&ds.chr_ram, nesle::kChrRamBytes * P);
        if (cfg.frames) {
            add(&ds.present, static_cast<std::size_t>(nesle::present::kHeader + ds.vram_stride) * n);
            add(&ds.lat_sx, n); add(&ds.lat_sy, n); add(&ds.lat_ctrl, n);
        }
        std::uint8_t* actions = nullptr;
        add(&actions, n);
        add(&ds.rewards, 4 * n); add(&ds.done, n); add(&ds.prev_x, 4 * n); add(&ds.prev_time, 4 * n);
        add(&d_obs, static_cast<std::size_t>(nesle::kRamBytes) * n);
        add(&d_mask, n);
        add(&d_blob, blob::kBytes);
        add(&d_levels, n);
        std::size_t total = 0;
        for (const auto& s : slots) total = align_up(total, 256) + s.bytes;
        hip_check(hipMalloc(&arena, total), "hipMalloc state arena");
        hip_check(hipMemsetAsync(arena, 0, total, stream), "hipMemsetAsync state arena");
        std::size_t off = 0;
        for (const auto& s : slots) {
            off = align_up(off, 256);
            *s.dst = static_cast<std::uint8_t*>(arena) + off;
            off += s.bytes;
        }
        ds.prg_ram = ds.ram + static_cast<std::size_t>(nesle::kRamBytes) * P;
        ds.actions = actions;
        ds.prg_rom = d_prg;
        ds.chr_rom = rom.chr.empty() ? nullptr : d_chr;
    }

    void ensure_stats() {
        if (stats_arena != nullptr) return;
        const std::size_t n = cfg.num_envs;
        const std::size_t a = align_up(8 * n, 256), b = align_up(4 * n, 256), c = align_up(4 * n, 256);
        const std::size_t total = a + b + c + 8 * 256 + 8 * 65536 + 8 * nesle::census::kCount;
        hip_check(hipMalloc(&stats_arena, total), "hipMalloc stats");
        // Counters read before the first statistics step read zero, not what
        // an earlier allocation left there (a kernel, not a memset, in case
        // the first request comes inside a stream capture).
        hip_check(nesle::launch_zero_u64(static_cast<unsigned long long*>(stats_arena),
                                         static_cast<std::uint32_t>(total / 8), stream),
                  "zero stats");
        auto* base = static_cast<std::uint8_t*>(stats_arena);
        ds.stat_instructions = reinterpret_cast<std::uint64_t*>(base);
        ds.stat_frames = reinterpret_cast<std::uint32_t*>(base + a);
        ds.stat_budget_hits = reinterpret_cast<std::uint32_t*>(base + a + b);
        ds.prof_opcodes = reinterpret_cast<unsigned long long*>(base + a + b + c);
        ds.prof_pcs = ds.prof_opcodes + 256;
        ds.census = ds.prof_pcs + 65536;
    }

    void refresh_obs() { hip_check(nesle::launch_ram_obs(ds, d_obs, stream), "ram_obs_kernel"); }

    // Presentation snapshot from live state (full resets, state loads).
    void seed_present(const std::uint8_t* dmask) {
        hip_check(nesle::launch_seed_present(ds, dmask, stream), "seed_present_kernel");
    }

    std::uint8_t* frame_buffer(int output) {
        const std::size_t n = cfg.num_envs;
        std::uint8_t** slot = output == NESLE_FRAME_RGB ? &d_frame_rgb
                              : output == NESLE_FRAME_PALETTE ? &d_frame_palette : &d_gray84;
        const std::size_t bytes = output == NESLE_FRAME_RGB ? n * 240 * 256 * 3
                                  : output == NESLE_FRAME_PALETTE ? n * 240 * 256
                                                                  : n * nesle::render::kOut * nesle::render::kOut;
        if (*slot == nullptr) hip_check(hipMalloc(slot, bytes), "hipMalloc frame buffer");
        return *slot;
    }

    void ensure_render_tables() {
        if (d_render_tables != nullptr) return;
        const nesle::render::Tables t = nesle::render::make_tables();
        hip_check(hipMalloc(&d_render_tables, sizeof(t)), "hipMalloc render tables");
        host_to_device(d_render_tables, &t, sizeof(t), "upload render tables");
    }

    static Marks new_marks() {
        Marks e{};
        hip_check(hipEventCreate(&e.start), "hipEventCreate");
        hip_check(hipEventCreate(&e.stepped), "hipEventCreate");
        hip_check(hipEventCreate(&e.reset), "hipEventCreate");
        return e;
    }

    Marks take_events() {
        if (spare.empty()) return new_marks();
        const Marks e = spare.back();
        spare.pop_back();
        return e;
    }

    // Fold completed event triples into the totals (all of them when `wait`).
    void fold_events(bool wait) {
        std::size_t done = 0;
        for (auto& e : events) {
            if (!wait && hipEventQuery(e.reset) != hipSuccess) break;
            hip_check(hipEventSynchronize(e.reset), "hipEventSynchronize");
            float step_ms = 0.0f, reset_ms = 0.0f;
            hip_check(hipEventElapsedTime(&step_ms, e.start, e.stepped), "hipEventElapsedTime");
            // A step without auto-reset launches no restore kernel: the gap
            // between its two events is event overhead, not kernel time.
            if (e.restored) hip_check(hipEventElapsedTime(&reset_ms, e.stepped, e.reset), "hipEventElapsedTime");
            timed_ms += step_ms;
            timed_reset_ms += reset_ms;
            ++timed_launches;
            spare.push_back(e);
            ++done;
        }
        events.erase(events.begin(), events.begin() + static_cast<std::ptrdiff_t>(done));
    }

    void grow_bank(std::uint32_t want) {
        if (want <= bank_capacity) return;
        std::uint32_t cap = std::max<std::uint32_t>(want, bank_capacity * 2);
        cap = std::min<std::uint32_t>(std::max<std::uint32_t>(cap, 8), 255);
        if (want > cap) throw InvalidArgument("a batch holds at most 255 snapshot levels");
        std::uint8_t* nb = nullptr;
        hip_check(hipMalloc(&nb, static_cast<std::size_t>(cap) * blob::kBytes), "hipMalloc snapshot bank");
        if (d_bank != nullptr && num_levels != 0) {
            hip_check(hipMemcpyAsync(nb, d_bank, static_cast<std::size_t>(num_levels) * blob::kBytes,
                                     hipMemcpyDeviceToDevice, stream),
                      "copy snapshot bank");
            sync();
        }
        (void)hipFree(d_bank);
        d_bank = nb;
        bank_capacity = cap;
    }

    void host_to_device(void* dst, const void* src, std::size_t bytes, const char* what) {
        hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream), what);
        sync();  // the host buffer may be released right after return
    }
};

void nesle::set_last_error(const std::string& msg) { g_error = msg; }

extern "C" {

const char* nesle_last_error(void) { return g_error.c_str(); }

void nesle_config_init(nesle_config* cfg) {
    if (cfg == nullptr) return;
    std::memset(cfg, 0, sizeof(*cfg));
    cfg->frameskip = 4;
    cfg->max_instructions_per_frame = 200000;
    cfg->reward_kind = NESLE_REWARD_SMB;
    cfg->x_lo = 0x86;
    cfg->x_hi = 0x6D;
    cfg->done_addr = 0;
    cfg->clip = 15;
    cfg->device = -1;
    cfg->frames = 1;
}

int nesle_parse_ines(const std::uint8_t* bytes, std::size_t len, nesle_rom_info* out) {
    return guarded([&] {
        const Rom r = parse_ines(bytes, len);
        if (out != nullptr) *out = r.info;
    });
}

int nesle_parse_fcs(const std::uint8_t* bytes, std::size_t len, std::uint8_t* out_blob) {
    return guarded([&] {
        if (bytes == nullptr || out_blob == nullptr) throw InvalidArgument("null buffer");
        fcs_to_blob(bytes, len, out_blob);
    });
}

namespace {

void check_config(const nesle_config* cfg) {
    if (cfg->num_envs == 0) throw InvalidArgument("num_envs must be positive");
    if (cfg->num_envs > NESLE_MAX_ENVS)
        throw InvalidArgument("num_envs must be at most " + std::to_string(NESLE_MAX_ENVS));
    if (cfg->frameskip == 0) throw InvalidArgument("frameskip must be positive");
    if (cfg->reward_kind > NESLE_REWARD_XDELTA) throw InvalidArgument("unknown reward_kind");
}

// Allocate and power on a batch for `b->rom` (parsed and checked by the caller).
void open_batch(nesle_batch* b, const nesle_config* cfg) {
    int dev = cfg->device;
    if (dev < 0) hip_check(hipGetDevice(&dev), "hipGetDevice");
    b->device = dev;
    b->activate();
    b->pitch = static_cast<std::uint32_t>(align_up(cfg->num_envs, 256));
    DeviceState& s = b->ds;
    s.n = cfg->num_envs;
    s.pitch = b->pitch;
    s.nt_mode = b->rom.info.nametable_arrangement;
    s.nt_bytes = s.nt_mode == 2 ? 4096u : 2048u;
    s.vram_stride = nesle::vram::stride(s.nt_bytes);
    s.prg_mask = static_cast<std::uint32_t>(b->rom.prg.size() - 1);
    s.chr_size = static_cast<std::uint32_t>(b->rom.chr.size());
    s.reward_kind = b->cfg.reward_kind;
    s.x_lo = b->cfg.x_lo & 0x7FF;
    s.x_hi = b->cfg.x_hi & 0x7FF;
    s.done_addr = b->cfg.done_addr & 0x7FF;
    s.clip = b->cfg.clip;
    s.time_penalty = b->cfg.time_penalty;
    b->allocate();
    b->host_to_device(b->d_prg, b->rom.prg.data(), b->rom.prg.size(), "upload PRG ROM");
    if (!b->rom.chr.empty()) b->host_to_device(b->d_chr, b->rom.chr.data(), b->rom.chr.size(), "upload CHR ROM");
    hip_check(nesle::launch_reset(s, nullptr, b->stream), "reset_kernel");
    if (b->synthetic) {
        hip_check(hipMalloc(&b->d_step_counts, sizeof(std::uint32_t) * s.n), "hipMalloc step counts");
        hip_check(nesle::launch_synthetic_reset(s, nullptr, b->d_step_counts, b->stream), "synthetic_reset_kernel");
    }
    b->seed_present(nullptr);
    b->refresh_obs();
    b->sync();
}

}  // namespace

int nesle_create(const nesle_config* cfg, const std::uint8_t* ines, std::size_t ines_len, nesle_batch** out) {
    return guarded([&] {
        if (out == nullptr || cfg == nullptr) throw InvalidArgument("null argument");
        *out = nullptr;
        check_config(cfg);
        auto b = std::make_unique<nesle_batch>();
        b->cfg = *cfg;
        if (b->cfg.max_instructions_per_frame == 0) b->cfg.max_instructions_per_frame = 200000;
        b->rom = parse_ines(ines, ines_len);
        if (b->rom.info.mapper != 0 || (b->rom.prg.size() != 16384 && b->rom.prg.size() != 32768))
            throw InvalidArgument("only mapper 0 (NROM) cartridges run on this console");
        open_batch(b.get(), cfg);
        *out = b.release();
    });
}

int nesle_create_synthetic(const nesle_config* cfg, nesle_batch** out) {
    return guarded([&] {
        if (out == nullptr || cfg == nullptr) throw InvalidArgument("null argument");
        *out = nullptr;
        check_config(cfg);
        auto b = std::make_unique<nesle_batch>();
        b->cfg = *cfg;
        b->cfg.reward_kind = NESLE_REWARD_SMB;   // the synthetic RAM is scored by the SMB rule only
        if (b->cfg.max_instructions_per_frame == 0) b->cfg.max_instructions_per_frame = 200000;
        b->synthetic = true;
        // No cartridge: an all-zero NROM-128 image stands in, so the batch's
        // memory map, views and (blank) frames exist; no console ever runs it.
        b->rom.info.prg_rom_size = 16384;
        b->rom.info.chr_rom_size = 8192;
        b->rom.prg.assign(16384, 0);
        b->rom.chr.assign(8192, 0);
        open_batch(b.get(), &b->cfg);
        *out = b.release();
    });
}

int nesle_synthetic_step(nesle_batch* b, int apply_actions, int auto_reset) {
    return guarded([&] {
        if (b == nullptr) throw InvalidArgument("null batch");
        if (!b->synthetic) throw InvalidArgument("nesle_synthetic_step needs a batch from nesle_create_synthetic");
        b->activate();
        hip_check(nesle::launch_synthetic_step(b->ds, b->cfg.frameskip, b->d_step_counts, apply_actions != 0, b->stream),
                  "synthetic_step_kernel");
        if (auto_reset != 0)
            hip_check(nesle::launch_synthetic_reset(b->ds, b->ds.done, b->d_step_counts, b->stream),
                      "synthetic_reset_kernel");
        b->refresh_obs();
    });
}

int nesle_set_snapshots(nesle_batch* b, const std::uint8_t* const* blobs, const std::size_t* lens, std::uint32_t count,
                        const std::uint8_t* env_to_level) {
    return guarded([&] {
        if (b == nullptr) throw InvalidArgument("null batch");
        if (b->synthetic) throw InvalidArgument("the ROM-less synthetic batch takes no snapshots");
        if (count == 0) throw InvalidArgument("the snapshot list is empty: give at least one snapshot");
        if (count > 255) throw InvalidArgument("a batch holds at most 255 snapshot levels");
        std::vector<std::uint8_t> host(static_cast<std::size_t>(count) * blob::kBytes);
        for (std::uint32_t i = 0; i < count; ++i) {
            if (blobs[i] == nullptr) throw InvalidArgument("null snapshot");
            const auto c = to_canonical(blobs[i], lens[i]);
            std::memcpy(host.data() + static_cast<std::size_t>(i) * blob::kBytes, c.data(), blob::kBytes);
        }
        std::vector<std::uint8_t> levels(b->n(), 0);
        if (env_to_level != nullptr) {
            for (std::uint32_t e = 0; e < b->n(); ++e) {
                if (env_to_level[e] >= count)
                    throw InvalidArgument("env_to_level[" + std::to_string(e) + "]=" + std::to_string(env_to_level[e]) +
                                          " out of range (have " + std::to_string(count) + " levels)");
                levels[e] = env_to_level[e];
            }
        }
        b->activate();
        b->num_levels = 0;
        b->grow_bank(count);
        b->host_to_device(b->d_bank, host.data(), host.size(), "upload snapshot bank");
        b->host_to_device(b->d_levels, levels.data(), levels.size(), "upload env_to_level");
        b->num_levels = count;
        b->ds.bank = b->d_bank;
        b->ds.env_to_level = b->d_levels;
        b->ds.num_levels = count;
        hip_check(nesle::launch_reset(b->ds, nullptr, b->stream), "reset_kernel");
        b->seed_present(nullptr);
        b->refresh_obs();
        b->sync();
    });
}

void nesle_retain(nesle_batch* b) {
    if (b != nullptr) b->refs.fetch_add(1);
}

void nesle_release(nesle_batch* b) {
    if (b != nullptr && b->refs.fetch_sub(1) == 1) delete b;
}

int nesle_reset(nesle_batch* b) {
    return guarded([&] {
        if (b == nullptr) throw InvalidArgument("null batch");
        b->activate();
        if (b->synthetic)
            hip_check(nesle::launch_synthetic_reset(b->ds, nullptr, b->d_step_counts, b->stream), "synthetic_reset_kernel");
        else
            hip_check(nesle::launch_reset(b->ds, nullptr, b->stream), "reset_kernel");
        b->seed_present(nullptr);
        b->refresh_obs();
        b->sync();
    });
}

int nesle_reset_envs(nesle_batch* b, const std::uint8_t* mask, int mask_on_device) {
    return guarded([&] {
        if (b == nullptr || mask == nullptr) throw InvalidArgument("null argument");
        b->activate();
        const std::uint8_t* dmask = mask;
        if (!mask_on_device) {
            b->host_to_device(b->d_mask, mask, b->n(), "copy reset mask");
            dmask = b->d_mask;
        }
        if (b->synthetic)
            hip_check(nesle::launch_synthetic_reset(b->ds, dmask, b->d_step_counts, b->stream), "synthetic_reset_kernel");
        else
            hip_check(nesle::launch_reset(b->ds, dmask, b->stream), "reset_kernel");
        b->refresh_obs();
        if (!mask_on_device) b->sync();   // a device mask stays ordered on the stream
    });
}

int nesle_set_actions(nesle_batch* b, const void* actions, int dtype, int on_device) {
    return guarded([&] {
        if (b == nullptr || actions == nullptr) throw InvalidArgument("null argument");
        b->activate();
        auto* dst = const_cast<std::uint8_t*>(b->ds.actions);
        const std::size_t n = b->n();
        if (dtype == NESLE_DTYPE_U8) {
            if (on_device) {
                hip_check(hipMemcpyAsync(dst, actions, n, hipMemcpyDeviceToDevice, b->stream), "copy actions");
            } else {
                b->host_to_device(dst, actions, n, "copy actions");
            }
        } else if (dtype == NESLE_DTYPE_I64) {
            if (on_device) {
                hip_check(nesle::launch_actions_i64(dst, static_cast<const long long*>(actions), b->n(), b->stream),
                          "actions_i64_kernel");
            } else {
                std::vector<std::uint8_t> tmp(n);
                const auto* src = static_cast<const long long*>(actions);
                for (std::size_t i = 0; i < n; ++i) tmp[i] = static_cast<std::uint8_t>(src[i] & 0xFF);
                b->host_to_device(dst, tmp.data(), n, "copy actions");
            }
        } else {
            throw InvalidArgument("actions must be uint8 masks or int64 values already encoded as masks");
        }
    });
}

int nesle_step(nesle_batch* b, int auto_reset, int stats_mode) {
    return guarded([&] {
        if (b == nullptr) throw InvalidArgument("null batch");
        if (stats_mode < 0 || stats_mode > 3) throw InvalidArgument("stats_mode must be 0, 1, 2 or 3");
        if (b->synthetic) {   // no console runs: no instruction statistics (cuda_module.cu:667-670)
            if (stats_mode != 0) throw std::runtime_error("step statistics need a console batch (one made from a ROM)");
            b->activate();
            hip_check(nesle::launch_synthetic_step(b->ds, b->cfg.frameskip, b->d_step_counts, true, b->stream),
                      "synthetic_step_kernel");
            if (auto_reset != 0)
                hip_check(nesle::launch_synthetic_reset(b->ds, b->ds.done, b->d_step_counts, b->stream),
                          "synthetic_reset_kernel");
            b->refresh_obs();
            return;
        }
        b->activate();
        if (stats_mode != 0) {
            b->ensure_stats();
            if (stats_mode == 2) {
                // Opcode and PC histograms are contiguous.
                hip_check(nesle::launch_zero_u64(b->ds.prof_opcodes, 256 + 65536, b->stream), "clear profile");
            }
            if (stats_mode == 3)
                hip_check(nesle::launch_zero_u64(b->ds.census, nesle::census::kCount, b->stream), "clear census");
        }
        DeviceState s = b->ds;
        if (stats_mode == 0) {
            s.stat_instructions = nullptr;
            s.stat_frames = nullptr;
            s.stat_budget_hits = nullptr;
        }
        if (stats_mode != 2) {
            s.prof_opcodes = nullptr;
            s.prof_pcs = nullptr;
        }
        if (stats_mode != 3) s.census = nullptr;
        nesle_batch::Marks ev{};
        if (b->timing) {
            b->fold_events(false);
            ev = b->take_events();
            hip_check(hipEventRecord(ev.start, b->stream), "hipEventRecord");
        }
        hip_check(nesle::launch_step(s, b->cfg.frameskip, b->cfg.max_instructions_per_frame, stats_mode, b->stream),
                  "step_kernel");
        if (b->timing) hip_check(hipEventRecord(ev.stepped, b->stream), "hipEventRecord");
        // Auto-reset: done consoles restored from their level's snapshot (or
        // powered on); rewards and dones of the step stay as written, as the
        // reference's last_rewards/last_done copies do (cuda_module.cu:635-656).
        if (auto_reset != 0) hip_check(nesle::launch_reset(s, s.done, b->stream), "restore_kernel");
        if (b->timing) {
            hip_check(hipEventRecord(ev.reset, b->stream), "hipEventRecord");
            ev.restored = auto_reset != 0;
            b->events.push_back(ev);
        }
        b->refresh_obs();
    });
}

int nesle_get_view(nesle_batch* b, int kind, nesle_view* out) {
    return guarded([&] {
        if (b == nullptr || out == nullptr) throw InvalidArgument("null argument");
        const std::int64_t n = b->n();
        nesle_view v{};
        v.device_id = b->device;
        v.ndim = 1;
        v.shape[0] = n;
        auto frame = [&](std::uint8_t* buf, std::int32_t ndim, std::int64_t h, std::int64_t w, std::int64_t c) {
            if (buf == nullptr) throw InvalidArgument("no frames yet: call nesle_render with this output first");
            v.data = buf; v.ndim = ndim; v.shape[1] = h; v.shape[2] = w; v.shape[3] = c; v.dtype = NESLE_DTYPE_U8;
        };
        switch (kind) {
            case NESLE_VIEW_RAM: v.data = b->d_obs; v.ndim = 2; v.shape[1] = nesle::kRamBytes; v.dtype = NESLE_DTYPE_U8; break;
            case NESLE_VIEW_REWARDS: v.data = b->ds.rewards; v.dtype = NESLE_DTYPE_F32; break;
            case NESLE_VIEW_DONES: v.data = b->ds.done; v.dtype = NESLE_DTYPE_U8; break;
            case NESLE_VIEW_ACTIONS: v.data = const_cast<std::uint8_t*>(b->ds.actions); v.dtype = NESLE_DTYPE_U8; break;
            case NESLE_VIEW_INSTRUCTIONS: b->ensure_stats(); v.data = b->ds.stat_instructions; v.dtype = NESLE_DTYPE_U64; break;
            case NESLE_VIEW_FRAMES: b->ensure_stats(); v.data = b->ds.stat_frames; v.dtype = NESLE_DTYPE_U32; break;
            case NESLE_VIEW_BUDGET_HITS: b->ensure_stats(); v.data = b->ds.stat_budget_hits; v.dtype = NESLE_DTYPE_U32; break;
            case NESLE_VIEW_OPCODES: b->ensure_stats(); v.data = b->ds.prof_opcodes; v.shape[0] = 256; v.dtype = NESLE_DTYPE_U64; break;
            case NESLE_VIEW_PCS: b->ensure_stats(); v.data = b->ds.prof_pcs; v.shape[0] = 65536; v.dtype = NESLE_DTYPE_U64; break;
            case NESLE_VIEW_PRESENT:
                if (b->ds.present == nullptr) throw InvalidArgument("frames are off for this batch (created with frames = 0)");
                v.data = b->ds.present; v.ndim = 2; v.shape[1] = nesle::present::kHeader + b->ds.vram_stride;
                v.dtype = NESLE_DTYPE_U8;
                break;
            case NESLE_VIEW_CENSUS: b->ensure_stats(); v.data = b->ds.census; v.shape[0] = nesle::census::kCount; v.dtype = NESLE_DTYPE_U64; break;
            case NESLE_VIEW_FRAME_RGB: frame(b->d_frame_rgb, 4, 240, 256, 3); break;
            case NESLE_VIEW_FRAME_PALETTE: frame(b->d_frame_palette, 3, 240, 256, 0); break;
            case NESLE_VIEW_GRAY84: frame(b->d_gray84, 3, nesle::render::kOut, nesle::render::kOut, 0); break;
            default: throw InvalidArgument("unknown view kind");
        }
        *out = v;
    });
}

int nesle_copy_to_host(nesle_batch* b, int kind, void* dst, std::size_t bytes) {
    return guarded([&] {
        if (b == nullptr || dst == nullptr) throw InvalidArgument("null argument");
        b->activate();
        if (kind == NESLE_VIEW_OAM) {
            const std::size_t n = b->n();
            if (bytes != n * nesle::kOamBytes) throw InvalidArgument("OAM copy needs num_envs * 256 bytes");
            hip_check(hipMemcpy2DAsync(dst, nesle::kOamBytes, b->ds.vram + nesle::vram::kOam, b->ds.vram_stride,
                                       nesle::kOamBytes, n, hipMemcpyDeviceToHost, b->stream),
                      "copy oam");
            b->sync();
            return;
        }
        nesle_view v{};
        if (nesle_get_view(b, kind, &v) != NESLE_OK) throw InvalidArgument(g_error);
        static const std::size_t kSize[] = {1, 8, 4, 4, 8};
        std::size_t want = kSize[v.dtype];
        for (int d = 0; d < v.ndim; ++d) want *= static_cast<std::size_t>(v.shape[d]);
        if (bytes != want) throw InvalidArgument("host buffer has " + std::to_string(bytes) + " bytes, view needs " +
                                                 std::to_string(want));
        hip_check(hipMemcpyAsync(dst, v.data, bytes, hipMemcpyDeviceToHost, b->stream), "copy view to host");
        b->sync();
    });
}

int nesle_render(nesle_batch* b, std::uint32_t outputs) {
    return guarded([&] {
        if (b == nullptr) throw InvalidArgument("null batch");
        const std::uint32_t frames = outputs & (NESLE_FRAME_RGB | NESLE_FRAME_PALETTE | NESLE_FRAME_GRAY84);
        if (frames == 0 || (outputs & ~(frames | NESLE_FRAME_LIVE)) != 0)
            throw InvalidArgument("outputs must be a non-empty set of NESLE_FRAME_* output bits, optionally with NESLE_FRAME_LIVE");
        if (b->ds.present == nullptr) throw InvalidArgument("frames are off for this batch (created with frames = 0)");
        b->activate();
        b->ensure_render_tables();
        nesle::RenderArgs a{};
        a.n = b->n();
        a.present = b->ds.present;
        a.present_stride = nesle::present::kHeader + b->ds.vram_stride;
        if (outputs & NESLE_FRAME_LIVE) {
            if (b->d_live_records == nullptr)
                hip_check(hipMalloc(&b->d_live_records, static_cast<std::size_t>(a.n) * a.present_stride),
                          "hipMalloc live records");
            hip_check(nesle::launch_live_records(b->ds, b->d_live_records, b->stream), "record_kernel");
            a.present = b->d_live_records;
            a.cpu_rules = 1;
            a.chr_ram = b->ds.chr_ram;
            a.pitch = b->ds.pitch;
        }
        a.chr = b->rom.chr.empty() ? nullptr : b->d_chr;
        a.chr_size = static_cast<std::uint32_t>(b->rom.chr.size());
        a.nt_mode = b->ds.nt_mode;
        a.tables = static_cast<const nesle::render::Tables*>(b->d_render_tables);
        a.rgb = (outputs & NESLE_FRAME_RGB) ? b->frame_buffer(NESLE_FRAME_RGB) : nullptr;
        a.palette = (outputs & NESLE_FRAME_PALETTE) ? b->frame_buffer(NESLE_FRAME_PALETTE) : nullptr;
        a.gray = (outputs & NESLE_FRAME_GRAY84) ? b->frame_buffer(NESLE_FRAME_GRAY84) : nullptr;
        hip_check(nesle::launch_render(a, b->stream), "render_kernel");
    });
}

int nesle_save_state(nesle_batch* b, std::uint32_t env, std::uint8_t* out_blob) {
    return guarded([&] {
        if (b == nullptr || out_blob == nullptr) throw InvalidArgument("null argument");
        if (env >= b->n()) throw InvalidArgument("env out of range");
        b->activate();
        hip_check(nesle::launch_save_blob(b->ds, env, b->d_blob, b->stream), "save_blob_kernel");
        hip_check(hipMemcpyAsync(out_blob, b->d_blob, blob::kBytes, hipMemcpyDeviceToHost, b->stream), "copy state");
        b->sync();
    });
}

int nesle_load_state(nesle_batch* b, const std::uint8_t* data, std::size_t len, const std::uint8_t* mask) {
    return guarded([&] {
        if (b == nullptr || data == nullptr) throw InvalidArgument("null argument");
        if (b->synthetic) throw InvalidArgument("the ROM-less synthetic batch has no console state to load");
        b->activate();
        const auto c = to_canonical(data, len);
        b->host_to_device(b->d_blob, c.data(), c.size(), "upload state");
        const std::uint8_t* dmask = nullptr;
        if (mask != nullptr) {
            b->host_to_device(b->d_mask, mask, b->n(), "upload mask");
            dmask = b->d_mask;
        }
        hip_check(nesle::launch_load_blob(b->ds, b->d_blob, dmask, b->stream), "load_blob_kernel");
        b->seed_present(dmask);
        b->refresh_obs();
        b->sync();
    });
}

int nesle_snapshot_capture(nesle_batch* b, std::uint32_t env, std::uint32_t slot) {
    return guarded([&] {
        if (b == nullptr) throw InvalidArgument("null batch");
        if (b->synthetic) throw InvalidArgument("the ROM-less synthetic batch takes no snapshots");
        if (env >= b->n()) throw InvalidArgument("env out of range");
        if (slot > b->num_levels) throw InvalidArgument("slot must be an existing level or the next free one");
        b->activate();
        b->grow_bank(slot + 1);
        hip_check(nesle::launch_save_blob(b->ds, env, b->d_bank + static_cast<std::size_t>(slot) * blob::kBytes,
                                          b->stream),
                  "save_blob_kernel");
        if (slot == b->num_levels) ++b->num_levels;
        b->ds.bank = b->d_bank;
        b->ds.env_to_level = b->d_levels;
        b->ds.num_levels = b->num_levels;
        b->sync();
    });
}

int nesle_snapshot_export(nesle_batch* b, std::uint32_t slot, std::uint8_t* out_blob) {
    return guarded([&] {
        if (b == nullptr || out_blob == nullptr) throw InvalidArgument("null argument");
        if (slot >= b->num_levels) throw InvalidArgument("slot out of range");
        b->activate();
        hip_check(hipMemcpyAsync(out_blob, b->d_bank + static_cast<std::size_t>(slot) * blob::kBytes, blob::kBytes,
                                 hipMemcpyDeviceToHost, b->stream),
                  "copy snapshot");
        b->sync();
    });
}

int nesle_set_env_levels(nesle_batch* b, const std::uint8_t* env_to_level) {
    return guarded([&] {
        if (b == nullptr || env_to_level == nullptr) throw InvalidArgument("null argument");
        for (std::uint32_t e = 0; e < b->n(); ++e)
            if (env_to_level[e] >= b->num_levels)
                throw InvalidArgument("env_to_level[" + std::to_string(e) + "] out of range");
        b->activate();
        b->host_to_device(b->d_levels, env_to_level, b->n(), "upload env_to_level");
    });
}

int nesle_poke_ram(nesle_batch* b, std::uint32_t address, std::uint32_t value) {
    return guarded([&] {
        if (b == nullptr) throw InvalidArgument("null batch");
        b->activate();
        hip_check(nesle::launch_poke_ram(b->ds, address, value & 0xFF, b->stream), "poke_ram_kernel");
        b->refresh_obs();
        b->sync();
    });
}

int nesle_poke_ram_envs(nesle_batch* b, std::uint32_t address, const std::uint8_t* values, int on_device) {
    return guarded([&] {
        if (b == nullptr || values == nullptr) throw InvalidArgument("null argument");
        b->activate();
        const std::uint8_t* dv = values;
        if (!on_device) {
            b->host_to_device(b->d_mask, values, b->n(), "copy RAM values");
            dv = b->d_mask;
        }
        hip_check(nesle::launch_poke_ram_envs(b->ds, address, dv, b->stream), "poke_ram_envs_kernel");
        b->refresh_obs();
        if (!on_device) b->sync();   // the staging buffer is reused by the next call
    });
}

int nesle_synchronize(nesle_batch* b) {
    return guarded([&] {
        if (b == nullptr) throw InvalidArgument("null batch");
        b->activate();
        b->sync();
    });
}

int nesle_set_stream(nesle_batch* b, void* hip_stream) {
    return guarded([&] {
        if (b == nullptr) throw InvalidArgument("null batch");
        b->sync();
        b->stream = static_cast<hipStream_t>(hip_stream);
    });
}

int nesle_set_timing(nesle_batch* b, int enable) {
    return guarded([&] {
        if (b == nullptr) throw InvalidArgument("null batch");
        b->activate();
        b->fold_events(true);
        b->timing = enable != 0;
        b->timed_ms = 0.0;
        b->timed_reset_ms = 0.0;
        b->timed_launches = 0;
        // Events for the first timed steps exist before they are recorded.
        while (b->timing && b->spare.size() < 4) b->spare.push_back(nesle_batch::new_marks());
    });
}

int nesle_get_timing(nesle_batch* b, double* total_ms, std::uint64_t* launches) {
    return nesle_get_timing_split(b, total_ms, nullptr, launches);
}

int nesle_get_timing_split(nesle_batch* b, double* step_ms, double* reset_ms, std::uint64_t* launches) {
    return guarded([&] {
        if (b == nullptr) throw InvalidArgument("null batch");
        b->activate();
        b->fold_events(true);
        if (step_ms != nullptr) *step_ms = b->timed_ms;
        if (reset_ms != nullptr) *reset_ms = b->timed_reset_ms;
        if (launches != nullptr) *launches = b->timed_launches;
    });
}

std::uint32_t nesle_num_envs(const nesle_batch* b) { return b ? b->cfg.num_envs : 0; }
std::uint32_t nesle_frameskip(const nesle_batch* b) { return b ? b->cfg.frameskip : 0; }
std::uint32_t nesle_num_levels(const nesle_batch* b) { return b ? b->num_levels : 0; }
std::int32_t nesle_device_id(const nesle_batch* b) { return b ? b->device : -1; }

}  // extern "C"
