// nes_render.hip -- frames of the batched console: palette-value, RGB and
// 84x84 gray observations from the presentation snapshot.
//
// Semantics are the batched core's renderer (cpp/include/nesle/cuda/
// batch_render.cuh:161-440): each pixel takes the background of the snapshot
// (rows above sprite 0's bottom edge use the frame-start scroll/ctrl, the rest
// the frame-end values; with sprite 0 off screen the whole frame uses the
// frame-start values), a background pixel whose palette value is 0 counts as
// transparent, CHR RAM reads as 0, and the lowest-index sprite that is opaque
// and not behind an opaque background pixel wins.  RGB uses the renderer's
// 64-entry palette.  The gray observation is the pixel preprocessing of the
// reference's training project (project/mario-rl-ram/src/mario_rl/
// wrappers.py:209-215): luma truncated to 8 bits, then Pillow's BILINEAR
// resize to 84x84; the host computes its fixed-point weights (nes_render.h).
//
// One workgroup of 256 threads renders one console in bands of 8 rows: each
// thread owns one x column, writes the requested full-size outputs (coalesced
// across threads) and the band feeds the horizontal resample pass in LDS; the
// vertical pass runs once the 240 x 84 intermediate is complete.  Every
// console reads the same 8 KB of CHR ROM, so each workgroup stages it in LDS.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "nes_layout.h"
#include "nes_render.h"

namespace nesle {
namespace {

constexpr std::uint32_t kThreads = 256;
constexpr std::uint32_t kBand = 8;

struct View {
    std::uint32_t ctrl, sx, sy;
};

struct Frame {
    const std::uint8_t* chr;   // LDS, chr_size bytes (0 => CHR RAM, reads 0)
    std::uint32_t chr_size, nt_mode, mask;
    const std::uint8_t* nt;    // LDS snapshot nametables
    const std::uint8_t* pal;   // LDS snapshot palette
    const std::uint8_t* oam;   // LDS snapshot OAM

    __device__ std::uint32_t nt_index(std::uint32_t addr) const {
        const std::uint32_t i = (addr - 0x2000) & 0x0FFF;
        if (nt_mode == 2) return i;
        if (nt_mode == 0) return i & 0x07FF;
        return (i & 0x03FF) | ((i & 0x0800) >> 1);
    }
    // batch_ppu_memory_read (batch_render.cuh:103-122).
    __device__ std::uint32_t read(std::uint32_t addr) const {
        addr &= 0x3FFF;
        if (addr < 0x2000) return chr_size != 0 ? chr[addr % chr_size] : 0u;
        if (addr < 0x3F00) {
            if (addr >= 0x3000) addr -= 0x1000;
            return nt[nt_index(addr)];
        }
        std::uint32_t i = addr & 0x1F;
        if ((i & 0x13) == 0x10) i &= 0x0F;
        return pal[i];
    }
    __device__ std::uint32_t palette_value(std::uint32_t index) const {
        std::uint32_t v = read(0x3F00 + index);
        if (mask & 0x01) v &= 0x30;
        return v & 0x3F;
    }
    __device__ std::uint32_t pattern(std::uint32_t tile_base, std::uint32_t fx, std::uint32_t fy) const {
        const std::uint32_t lo = read(tile_base + fy), hi = read(tile_base + fy + 8);
        const std::uint32_t bit = 7 - fx;
        return ((lo >> bit) & 1) | (((hi >> bit) & 1) << 1);
    }
    // batch_background_color: the palette value, 0 when transparent.
    __device__ std::uint32_t background(const View& w, std::uint32_t x, std::uint32_t y) const {
        if (!(mask & 0x08) || (!(mask & 0x02) && x < 8)) return 0;
        const std::uint32_t wy = w.sy + y, wx = w.sx + x;
        const std::uint32_t coarse_y = (wy % 240) / 8, fine_y = wy & 7;
        const std::uint32_t base_nt = w.ctrl & 3;
        const std::uint32_t nt_y = ((base_nt >> 1) + wy / 240) & 1;
        const std::uint32_t coarse_x = (wx & 0xFF) / 8, fine_x = wx & 7;
        const std::uint32_t nt_x = ((base_nt & 1) + wx / 256) & 1;
        const std::uint32_t nt_base = 0x2000 + (nt_x | (nt_y << 1)) * 0x400;
        const std::uint32_t tile = read(nt_base + coarse_y * 32 + coarse_x);
        const std::uint32_t c = pattern(((w.ctrl & 0x10) ? 0x1000u : 0u) + tile * 16, fine_x, fine_y);
        if (c == 0) return 0;
        const std::uint32_t attr = read(nt_base + 0x3C0 + (coarse_y / 4) * 8 + coarse_x / 4);
        const std::uint32_t shift = ((coarse_y & 2) << 1) | (coarse_x & 2);
        return palette_value(((attr >> shift) & 3) * 4 + c);
    }
    // batch_sprite_pattern_pixel.
    __device__ std::uint32_t sprite(std::uint32_t ctrl, std::uint32_t tile, std::uint32_t attr, std::uint32_t px,
                                    std::uint32_t py) const {
        if (attr & 0x40) px = 7 - px;
        if (ctrl & 0x20) {
            if (attr & 0x80) py = 15 - py;
            const std::uint32_t t = ((tile & 0xFE) + py / 8) & 0xFF;
            return pattern(((tile & 1) ? 0x1000u : 0u) + t * 16, px, py & 7);
        }
        if (attr & 0x80) py = 7 - py;
        return pattern(((ctrl & 0x08) ? 0x1000u : 0u) + tile * 16, px, py);
    }
};

__constant__ std::uint8_t c_nes_rgb[192] = {
    0x54, 0x54, 0x54, 0x00, 0x1E, 0x74, 0x08, 0x10, 0x90, 0x30, 0x00, 0x88,
    0x44, 0x00, 0x64, 0x5C, 0x00, 0x30, 0x54, 0x04, 0x00, 0x3C, 0x18, 0x00,
    0x20, 0x2A, 0x00, 0x08, 0x3A, 0x00, 0x00, 0x40, 0x00, 0x00, 0x3C, 0x00,
    0x00, 0x32, 0x3C, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00,
    0x98, 0x96, 0x98, 0x08, 0x4C, 0xC4, 0x30, 0x32, 0xEC, 0x5C, 0x1E, 0xE4,
    0x88, 0x14, 0xB0, 0xA0, 0x14, 0x64, 0x98, 0x22, 0x20, 0x78, 0x3C, 0x00,
    0x54, 0x5A, 0x00, 0x28, 0x72, 0x00, 0x08, 0x7C, 0x00, 0x00, 0x76, 0x28,
    0x00, 0x66, 0x78, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00,
    0xEC, 0xEE, 0xEC, 0x4C, 0x9A, 0xEC, 0x78, 0x7C, 0xEC, 0xB0, 0x62, 0xEC,
    0xE4, 0x54, 0xEC, 0xEC, 0x58, 0xB4, 0xEC, 0x6A, 0x64, 0xD4, 0x88, 0x20,
    0xA0, 0xAA, 0x00, 0x74, 0xC4, 0x00, 0x4C, 0xD0, 0x20, 0x38, 0xCC, 0x6C,
    0x38, 0xB4, 0xCC, 0x3C, 0x3C, 0x3C, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00,
    0xEC, 0xEE, 0xEC, 0xA8, 0xCC, 0xEC, 0xBC, 0xBC, 0xEC, 0xD4, 0xB2, 0xEC,
    0xEC, 0xAE, 0xEC, 0xEC, 0xAE, 0xD4, 0xEC, 0xB4, 0xB0, 0xE4, 0xC4, 0x90,
    0xCC, 0xD2, 0x78, 0xB4, 0xDE, 0x78, 0xA8, 0xE2, 0x90, 0x98, 0xE2, 0xB4,
    0xA0, 0xD6, 0xE4, 0xA0, 0xA2, 0xA0, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00,
};

__device__ __forceinline__ std::uint32_t clip8(std::int32_t acc) {
    const std::int32_t v = acc >> render::kPrecision;
    return static_cast<std::uint32_t>(v < 0 ? 0 : (v > 255 ? 255 : v));
}

__global__ void __launch_bounds__(kThreads) render_kernel(RenderArgs a) {
    __shared__ __attribute__((aligned(16))) std::uint8_t chr[8192];
    __shared__ __attribute__((aligned(16))) std::uint8_t rec[present::kMaxBytes];
    __shared__ std::uint64_t rows[240];
    __shared__ std::uint8_t band[kBand][256];
    __shared__ std::uint8_t mid[240][render::kOut];
    __shared__ std::uint8_t gray_lut[64];
    __shared__ render::Taps taps;

    const std::uint32_t tid = threadIdx.x, env = blockIdx.x;
    {
        const uint4* src = reinterpret_cast<const uint4*>(a.present + static_cast<std::size_t>(env) * a.present_stride);
        for (std::uint32_t i = tid; i < a.present_stride / 16; i += kThreads) reinterpret_cast<uint4*>(rec)[i] = src[i];
        if (a.chr_size != 0) {
            const uint4* c = reinterpret_cast<const uint4*>(a.chr);
            for (std::uint32_t i = tid; i < 8192 / 16; i += kThreads) reinterpret_cast<uint4*>(chr)[i] = c[i % (a.chr_size / 16)];
        }
        if (tid < 64) gray_lut[tid] = a.gray_lut[tid];
        const std::uint32_t* t = reinterpret_cast<const std::uint32_t*>(a.taps);
        for (std::uint32_t i = tid; i < sizeof(render::Taps) / 4; i += kThreads) reinterpret_cast<std::uint32_t*>(&taps)[i] = t[i];
    }
    __syncthreads();

    Frame f{chr, a.chr_size != 0 ? (a.chr_size < 8192 ? a.chr_size : 8192u) : 0u, a.nt_mode, rec[present::kMask],
            rec + present::kNametable, rec + present::kPalette, rec + present::kOam};
    // resolve_render_env_views (batch_render.cuh:336-366).
    View play{rec[present::kCtrlEnd], rec[present::kSxEnd], rec[present::kSyEnd]};
    const View hud{rec[present::kCtrlStart], rec[present::kSxStart], rec[present::kSyStart]};
    std::int32_t split = static_cast<std::int32_t>(f.oam[0]) + 1 + ((play.ctrl & 0x20) ? 16 : 8);
    if (split >= 240) {
        play = hud;
        split = 0;
    }
    const std::uint32_t height = (play.ctrl & 0x20) ? 16 : 8;
    if (tid < 240) {   // sprites covering each row, by OAM index
        std::uint64_t m = 0;
        for (std::uint32_t s = 0; s < 64; ++s) {
            const std::uint32_t dy = tid - (static_cast<std::uint32_t>(f.oam[4 * s]) + 1);
            m |= (dy < height ? 1ull : 0ull) << s;
        }
        rows[tid] = m;
    }
    __syncthreads();

    const bool sprites = (f.mask & 0x10) != 0;
    const std::uint32_t x = tid;
    const bool sprite_col = sprites && ((f.mask & 0x04) || x >= 8);
    const std::uint32_t backdrop = f.palette_value(0);
    std::uint8_t* out_pal = a.palette ? a.palette + static_cast<std::size_t>(env) * 240 * 256 : nullptr;
    std::uint8_t* out_rgb = a.rgb ? a.rgb + static_cast<std::size_t>(env) * 240 * 256 * 3 : nullptr;
    for (std::uint32_t y0 = 0; y0 < 240; y0 += kBand) {
        for (std::uint32_t r = 0; r < kBand; ++r) {
            const std::uint32_t y = y0 + r;
            const View& bs = static_cast<std::int32_t>(y) < split ? hud : play;
            const std::uint32_t bgv = f.background(bs, x, y);
            std::uint32_t colour = bgv != 0 ? bgv : backdrop;
            std::uint64_t m = sprite_col ? rows[y] : 0ull;
            while (m != 0) {
                const std::uint32_t s = static_cast<std::uint32_t>(__ffsll(static_cast<long long>(m)) - 1);
                m &= m - 1;
                const std::uint32_t sx = x - f.oam[4 * s + 3];
                if (sx >= 8) continue;
                const std::uint32_t attr = f.oam[4 * s + 2];
                if ((attr & 0x20) && f.background(play, x, y) != 0) continue;
                const std::uint32_t sc = f.sprite(play.ctrl, f.oam[4 * s + 1], attr, sx, y - (f.oam[4 * s] + 1u));
                if (sc == 0) continue;
                colour = f.palette_value(0x10 + (attr & 3) * 4 + sc);
                break;
            }
            band[r][x] = static_cast<std::uint8_t>(colour);
            if (out_pal) out_pal[y * 256 + x] = static_cast<std::uint8_t>(colour);
            if (out_rgb) {
                std::uint8_t* o = out_rgb + (y * 256 + x) * 3;
                o[0] = c_nes_rgb[3 * colour]; o[1] = c_nes_rgb[3 * colour + 1]; o[2] = c_nes_rgb[3 * colour + 2];
            }
        }
        __syncthreads();
        if (a.gray) {   // horizontal pass of the band: 8 rows x 84 columns
            for (std::uint32_t i = tid; i < kBand * render::kOut; i += kThreads) {
                const std::uint32_t r = i / render::kOut, ox = i % render::kOut;
                std::int32_t acc = 1 << (render::kPrecision - 1);
                const std::uint32_t lo = taps.h_lo[ox], n = taps.h_n[ox];
                for (std::uint32_t j = 0; j < n; ++j) acc += gray_lut[band[r][lo + j]] * taps.h_k[ox][j];
                mid[y0 + r][ox] = static_cast<std::uint8_t>(clip8(acc));
            }
        }
        __syncthreads();
    }
    if (a.gray) {   // vertical pass
        std::uint8_t* out = a.gray + static_cast<std::size_t>(env) * render::kOut * render::kOut;
        for (std::uint32_t i = tid; i < render::kOut * render::kOut; i += kThreads) {
            const std::uint32_t oy = i / render::kOut, ox = i % render::kOut;
            std::int32_t acc = 1 << (render::kPrecision - 1);
            const std::uint32_t lo = taps.v_lo[oy], n = taps.v_n[oy];
            for (std::uint32_t j = 0; j < n; ++j) acc += mid[lo + j][ox] * taps.v_k[oy][j];
            out[i] = static_cast<std::uint8_t>(clip8(acc));
        }
    }
}

}  // namespace

// ---- host: resize weights and gray levels ------------------------------------
namespace render {
namespace {

constexpr std::uint8_t kNesRgbHost[192] = {
    0x54, 0x54, 0x54, 0x00, 0x1E, 0x74, 0x08, 0x10, 0x90, 0x30, 0x00, 0x88,
    0x44, 0x00, 0x64, 0x5C, 0x00, 0x30, 0x54, 0x04, 0x00, 0x3C, 0x18, 0x00,
    0x20, 0x2A, 0x00, 0x08, 0x3A, 0x00, 0x00, 0x40, 0x00, 0x00, 0x3C, 0x00,
    0x00, 0x32, 0x3C, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00,
    0x98, 0x96, 0x98, 0x08, 0x4C, 0xC4, 0x30, 0x32, 0xEC, 0x5C, 0x1E, 0xE4,
    0x88, 0x14, 0xB0, 0xA0, 0x14, 0x64, 0x98, 0x22, 0x20, 0x78, 0x3C, 0x00,
    0x54, 0x5A, 0x00, 0x28, 0x72, 0x00, 0x08, 0x7C, 0x00, 0x00, 0x76, 0x28,
    0x00, 0x66, 0x78, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00,
    0xEC, 0xEE, 0xEC, 0x4C, 0x9A, 0xEC, 0x78, 0x7C, 0xEC, 0xB0, 0x62, 0xEC,
    0xE4, 0x54, 0xEC, 0xEC, 0x58, 0xB4, 0xEC, 0x6A, 0x64, 0xD4, 0x88, 0x20,
    0xA0, 0xAA, 0x00, 0x74, 0xC4, 0x00, 0x4C, 0xD0, 0x20, 0x38, 0xCC, 0x6C,
    0x38, 0xB4, 0xCC, 0x3C, 0x3C, 0x3C, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00,
    0xEC, 0xEE, 0xEC, 0xA8, 0xCC, 0xEC, 0xBC, 0xBC, 0xEC, 0xD4, 0xB2, 0xEC,
    0xEC, 0xAE, 0xEC, 0xEC, 0xAE, 0xD4, 0xEC, 0xB4, 0xB0, 0xE4, 0xC4, 0x90,
    0xCC, 0xD2, 0x78, 0xB4, 0xDE, 0x78, 0xA8, 0xE2, 0x90, 0x98, 0xE2, 0xB4,
    0xA0, 0xD6, 0xE4, 0xA0, 0xA2, 0xA0, 0x00, 0x00, 0x00, 0x00, 0x00, 0x00,
};

// One axis of Pillow's separable resample: triangle filter (support 1)
// widened by the scale, weights normalised, then rounded to fixed point.
template <std::uint32_t kTaps>
void axis(int in_size, std::int32_t* lo, std::int32_t* n, std::int32_t (*k)[kTaps]) {
    const double scale = static_cast<double>(in_size) / kOut;
    const double filterscale = scale < 1.0 ? 1.0 : scale;
    const double support = filterscale;
    for (std::uint32_t xx = 0; xx < kOut; ++xx) {
        const double center = (xx + 0.5) * scale;
        const double ss = 1.0 / filterscale;
        int xmin = static_cast<int>(center - support + 0.5);
        if (xmin < 0) xmin = 0;
        int xmax = static_cast<int>(center + support + 0.5);
        if (xmax > in_size) xmax = in_size;
        xmax -= xmin;
        double w[kTaps] = {};
        double ww = 0.0;
        for (int x = 0; x < xmax; ++x) {
            double t = (x + xmin - center + 0.5) * ss;
            if (t < 0.0) t = -t;
            w[x] = t < 1.0 ? 1.0 - t : 0.0;
            ww += w[x];
        }
        for (std::uint32_t x = 0; x < kTaps; ++x) {
            if (static_cast<int>(x) < xmax && ww != 0.0) w[x] /= ww;
            k[xx][x] = static_cast<int>(x) < xmax
                           ? (w[x] < 0 ? static_cast<std::int32_t>(-0.5 + w[x] * (1 << kPrecision))
                                       : static_cast<std::int32_t>(0.5 + w[x] * (1 << kPrecision)))
                           : 0;
        }
        lo[xx] = xmin;
        n[xx] = xmax;
    }
}

}  // namespace

Taps make_taps() {
    Taps t{};
    axis<kHTaps>(256, t.h_lo, t.h_n, t.h_k);
    axis<kVTaps>(240, t.v_lo, t.v_n, t.v_k);
    return t;
}

void make_gray_lut(std::uint8_t* lut) {
    for (std::uint32_t c = 0; c < 64; ++c) {
        const double r = kNesRgbHost[3 * c], g = kNesRgbHost[3 * c + 1], b = kNesRgbHost[3 * c + 2];
        lut[c] = static_cast<std::uint8_t>(static_cast<int>(std::fma(b, 0.114, std::fma(g, 0.587, r * 0.299))));
    }
}

const std::uint8_t* nes_rgb() { return kNesRgbHost; }

}  // namespace render

hipError_t launch_render(const RenderArgs& a, hipStream_t stream) {
    if (a.n == 0) return hipSuccess;
    render_kernel<<<dim3(a.n), dim3(kThreads), 0, stream>>>(a);
    return hipGetLastError();
}

}  // namespace nesle
