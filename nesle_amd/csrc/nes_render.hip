// nes_render.hip -- frames of the batched console: palette-value, RGB and
// 84x84 gray observations from the presentation snapshot.
//
// Semantics are the batched core's renderer (cpp/include/nesle/cuda/
// batch_render.cuh:161-440): each pixel takes the background of the snapshot
// (rows above sprite 0's bottom edge use the frame-start scroll/ctrl, the rest
// the frame-end values; with sprite 0 off screen the whole frame uses the
// frame-start values), a background pixel whose palette value is 0 counts as
// transparent, CHR RAM reads as 0, and the lowest-index sprite that is opaque
// and not behind an opaque background pixel (of the frame-end view) wins.
// RGB uses the renderer's 64-entry palette.  The gray observation is the
// pixel preprocessing of the reference's training project (project/
// mario-rl-ram/src/mario_rl/wrappers.py:209-215): luma truncated to 8 bits,
// then Pillow's BILINEAR resize to 84x84; the host computes its fixed-point
// weights (nes_render.h).
//
// One workgroup of 256 threads renders one console in bands of 8 rows.  A
// thread owns 8 adjacent pixels of one row: it decodes the (at most two)
// background tiles under them once -- nametable byte, attribute, both pattern
// planes -- and then each sprite of the row that overlaps them once, so a
// tile fetch serves 8 pixels.  Full-size outputs are written as 8-byte runs
// (coalesced across the 32 threads of a row); the band's gray levels feed the
// horizontal resample pass in LDS and the vertical pass runs once the
// 240 x 84 intermediate is complete.  Pattern tables (8 KB, shared by every
// console) are staged in LDS per workgroup, zero-filled for CHR RAM.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "nes_layout.h"
#include "nes_render.h"

namespace nesle {
namespace {

constexpr std::uint32_t kThreads = 256;
constexpr std::uint32_t kBand = 8;
// Horizontally resampled rows kept for the vertical pass.  An output row is
// emitted after the first band that completes its input window; windows are
// at most 7 rows and end within the band, so no emitted row reaches back more
// than 14 rows and the next band overwrites only rows no pending output needs.
constexpr std::uint32_t kRing = 16;

// Scroll/ctrl pair one part of the frame is drawn with.
struct View {
    std::uint32_t ctrl, sx, sy;
};

// Reverse the bit order of a byte (pattern rows are stored leftmost pixel in bit 7).
__device__ __forceinline__ std::uint32_t rev8(std::uint32_t b) { return __builtin_bitreverse32(b) >> 24; }
// Bits 0-7 of b to the even bits 0, 2, ..., 14.
__device__ __forceinline__ std::uint32_t spread(std::uint32_t b) {
    b = (b | (b << 4)) & 0x0F0Fu;
    b = (b | (b << 2)) & 0x3333u;
    return (b | (b << 1)) & 0x5555u;
}

struct Console {
    const std::uint8_t* chr;   // LDS, 8 KB pattern tables
    const std::uint8_t* nt;    // LDS, snapshot nametable RAM
    const std::uint8_t* oam;   // LDS, snapshot OAM
    const std::uint8_t* pv;    // LDS, 32 palette values (aliases and grayscale applied)
    std::uint32_t mask;
    // Nametable n = x | y << 1 lives at (x * mx + y * my) * 0x400 of nametable
    // RAM: vertical mirroring mx = 1, my = 0; horizontal 0, 1; four-screen 1, 2.
    std::uint32_t mx, my;

    // Background of pixels x0..x0+7 of row y: palette values (0 = transparent)
    // packed 8 bits per pixel, two words.  batch_background_color
    // (batch_render.cuh:219-262) for each pixel, with one fetch per tile.
    __device__ void background(const View& w, std::uint32_t x0, std::uint32_t y, std::uint32_t out[2]) const {
        out[0] = out[1] = 0;
        if (!(mask & 0x08)) return;
        const std::uint32_t wy = w.sy + y;
        const std::uint32_t coarse_y = (wy % 240) >> 3, fine_y = wy & 7;
        const std::uint32_t nt_y = (((w.ctrl & 3) >> 1) + wy / 240) & 1;
        const std::uint32_t pbase = (w.ctrl & 0x10) ? 0x1000u : 0u;
        const std::uint32_t wx0 = w.sx + x0, fx = wx0 & 7;
        std::uint32_t planes = 0, pal = 0;   // 16 pattern pixels (2 bits each), 2 attribute selects
        for (std::uint32_t k = 0; k < 2; ++k) {
            const std::uint32_t wt = (wx0 >> 3) + k;                  // world tile column 0..63
            const std::uint32_t coarse_x = wt & 31;
            const std::uint32_t nt_x = ((w.ctrl & 1) + (wt >> 5)) & 1;
            const std::uint8_t* n = nt + (nt_x * mx + nt_y * my) * 0x400;
            const std::uint32_t tile = n[coarse_y * 32 + coarse_x];
            const std::uint32_t lo = chr[(pbase + tile * 16 + fine_y) & 0x1FFF];
            const std::uint32_t hi = chr[(pbase + tile * 16 + fine_y + 8) & 0x1FFF];
            const std::uint32_t attr = n[0x3C0 + (coarse_y >> 2) * 8 + (coarse_x >> 2)];
            const std::uint32_t shift = ((coarse_y & 2) << 1) | (coarse_x & 2);
            // Interleave the planes: pixel j of the tile (bit 7 - j of each
            // plane) at bits 2j..2j+1.
            planes |= (spread(rev8(lo)) | (spread(rev8(hi)) << 1)) << (16 * k);
            pal |= ((attr >> shift) & 3) << (2 * k);
        }
        // The 4 palette values of each tile's attribute, colour 0 cleared
        // (transparent); pixel i of the run is pixel fx + i of the pair.
        const std::uint32_t* pw = reinterpret_cast<const std::uint32_t*>(pv);
        const std::uint32_t p0 = pw[pal & 3] & ~0xFFu, p1 = pw[(pal >> 2) & 3] & ~0xFFu;
        const std::uint32_t run = planes >> (2 * fx);
        for (std::uint32_t i = 0; i < 8; ++i) {
            const std::uint32_t c = (run >> (2 * i)) & 3;
            const std::uint32_t v = ((i + fx < 8 ? p0 : p1) >> (8 * c)) & 0xFF;
            out[i >> 2] |= v << (8 * (i & 3));
        }
        if (!(mask & 0x02) && x0 == 0) out[0] = out[1] = 0;   // left 8 pixels hidden
    }
};

__device__ __forceinline__ std::uint32_t byte_of(const std::uint32_t w[2], std::uint32_t i) {
    return (w[i >> 2] >> (8 * (i & 3))) & 0xFF;
}

__device__ __forceinline__ std::uint32_t clip8(std::int32_t acc) {
    const std::int32_t v = acc >> render::kPrecision;
    return static_cast<std::uint32_t>(v < 0 ? 0 : (v > 255 ? 255 : v));
}

__global__ void __launch_bounds__(kThreads) render_kernel(RenderArgs a) {
    __shared__ __attribute__((aligned(16))) std::uint8_t chr[8192];
    __shared__ __attribute__((aligned(16))) std::uint8_t rec[present::kMaxBytes];
    __shared__ std::uint64_t rows[240];
    __shared__ __attribute__((aligned(16))) std::uint8_t gband[kBand][256];
    __shared__ std::uint8_t mid[kRing][render::kOut];
    __shared__ __attribute__((aligned(16))) render::Tables tab;
    __shared__ __attribute__((aligned(4))) std::uint8_t pv[32];

    const std::uint32_t tid = threadIdx.x, env = blockIdx.x;
    {
        const uint4* src = reinterpret_cast<const uint4*>(a.present + static_cast<std::size_t>(env) * a.present_stride);
        for (std::uint32_t i = tid; i < a.present_stride / 16; i += kThreads) reinterpret_cast<uint4*>(rec)[i] = src[i];
        // Pattern tables: the CHR ROM (an image smaller than 8 KB repeats), or
        // zeros for CHR RAM, which the batched renderer reads as 0.
        const std::uint32_t words = a.chr_size / 16;
        const uint4* c = reinterpret_cast<const uint4*>(a.chr);
        for (std::uint32_t i = tid; i < 8192 / 16; i += kThreads)
            reinterpret_cast<uint4*>(chr)[i] = words != 0 ? c[i % words] : make_uint4(0, 0, 0, 0);
        const std::uint32_t* t = reinterpret_cast<const std::uint32_t*>(a.tables);
        for (std::uint32_t i = tid; i < sizeof(render::Tables) / 4; i += kThreads)
            reinterpret_cast<std::uint32_t*>(&tab)[i] = t[i];
    }
    __syncthreads();

    const std::uint32_t mask = rec[present::kMask];
    const std::uint8_t* oam = rec + present::kOam;
    if (tid < 32) {   // batch_palette_value: aliases of $3F10/14/18/1C, grayscale, 6 bits
        const std::uint32_t i = ((tid & 0x13) == 0x10) ? (tid & 0x0F) : tid;
        std::uint32_t v = rec[present::kPalette + i];
        if (mask & 0x01) v &= 0x30;
        pv[tid] = static_cast<std::uint8_t>(v & 0x3F);
    }
    // resolve_render_env_views (batch_render.cuh:336-366).
    View play{rec[present::kCtrlEnd], rec[present::kSxEnd], rec[present::kSyEnd]};
    const View hud{rec[present::kCtrlStart], rec[present::kSxStart], rec[present::kSyStart]};
    std::int32_t split = static_cast<std::int32_t>(oam[0]) + 1 + ((play.ctrl & 0x20) ? 16 : 8);
    if (split >= 240) {
        play = hud;
        split = 0;
    }
    const std::uint32_t height = (play.ctrl & 0x20) ? 16 : 8;
    if (tid < 240) {   // sprites covering each row, by OAM index
        std::uint64_t m = 0;
        for (std::uint32_t s = 0; s < 64; ++s) {
            const std::uint32_t dy = tid - (static_cast<std::uint32_t>(oam[4 * s]) + 1);
            m |= (dy < height ? 1ull : 0ull) << s;
        }
        rows[tid] = (mask & 0x10) ? m : 0ull;
    }
    __syncthreads();

    Console con{chr, rec + present::kNametable, oam, pv, mask, a.nt_mode == 1 ? 0u : 1u,
                a.nt_mode == 2 ? 2u : a.nt_mode == 1 ? 1u : 0u};
    const std::uint32_t r = tid >> 5, x0 = (tid & 31) * 8;
    const std::uint32_t backdrop = pv[0];
    std::uint32_t next_oy = 0;   // first gray row not yet written
    // Horizontal resample: thread t < 252 owns output column t % 84 for band
    // rows t / 84, +3, +6, with that column's weights in registers (taps past
    // the window's end carry weight 0 and read inside the row).
    const std::uint32_t h_rows = tid < 3 * render::kOut ? 1u : 0u;
    const std::uint32_t h_ox = tid % render::kOut, h_r0 = tid / render::kOut;
    std::int32_t h_k[render::kHTaps];
    std::uint32_t h_lo = tab.taps.h_lo[h_ox];
    if (h_lo + render::kHTaps > 256) h_lo = 256 - render::kHTaps;
    for (std::uint32_t j = 0; j < render::kHTaps; ++j) {
        const std::int32_t k = static_cast<std::int32_t>(j + h_lo) - tab.taps.h_lo[h_ox];   // tap index of input h_lo + j
        h_k[j] = (k >= 0 && k < tab.taps.h_n[h_ox]) ? tab.taps.h_k[h_ox][k] : 0;
    }
    for (std::uint32_t y0 = 0; y0 < 240; y0 += kBand) {
        const std::uint32_t y = y0 + r;
        const bool upper = static_cast<std::int32_t>(y) < split;
        std::uint32_t bg[2];
        con.background(upper ? hud : play, x0, y, bg);
        std::uint32_t out[2] = {0, 0};
        for (std::uint32_t i = 0; i < 8; ++i) {
            const std::uint32_t v = byte_of(bg, i);
            out[i >> 2] |= (v != 0 ? v : backdrop) << (8 * (i & 3));
        }
        // Sprites, lowest OAM index first (batch_render.cuh:264-330).
        std::uint64_t m = rows[y];
        std::uint32_t done = ((mask & 0x04) || x0 >= 8) ? 0u : 0xFFu;   // left-column clipping
        bool have_play_bg = !upper;
        std::uint32_t play_bg[2] = {bg[0], bg[1]};
        while (m != 0 && done != 0xFF) {
            const std::uint32_t s = static_cast<std::uint32_t>(__ffsll(static_cast<long long>(m)) - 1);
            m &= m - 1;
            const std::uint32_t sxp = oam[4 * s + 3];
            const std::uint32_t off = x0 + 8 - sxp;   // sprite column of pixel i is i + x0 - sxp
            if (off - 1 >= 15) continue;              // no overlap with x0..x0+7
            const std::uint32_t attr = oam[4 * s + 2], tile = oam[4 * s + 1];
            std::uint32_t py = y - (oam[4 * s] + 1u);
            std::uint32_t addr;
            if (play.ctrl & 0x20) {
                if (attr & 0x80) py = 15 - py;
                addr = ((tile & 1) ? 0x1000u : 0u) + (((tile & 0xFE) + (py >> 3)) & 0xFF) * 16 + (py & 7);
            } else {
                if (attr & 0x80) py = 7 - py;
                addr = ((play.ctrl & 0x08) ? 0x1000u : 0u) + tile * 16 + py;
            }
            std::uint32_t lo = chr[addr & 0x1FFF], hi = chr[(addr + 8) & 0x1FFF];
            if (attr & 0x40) {
                lo = rev8(lo);
                hi = rev8(hi);
            }
            if ((attr & 0x20) && !have_play_bg) {   // behind: opacity of the frame-end view
                con.background(play, x0, y, play_bg);
                have_play_bg = true;
            }
            const std::uint32_t base = 0x10 + (attr & 3) * 4;
            for (std::uint32_t i = 0; i < 8; ++i) {
                const std::uint32_t px = i + x0 - sxp;
                if (px >= 8 || ((done >> i) & 1)) continue;
                const std::uint32_t bit = 7 - px;
                const std::uint32_t sc = ((lo >> bit) & 1) | (((hi >> bit) & 1) << 1);
                if (sc == 0 || ((attr & 0x20) && byte_of(play_bg, i) != 0)) continue;
                const std::uint32_t sh = 8 * (i & 3);
                out[i >> 2] = (out[i >> 2] & ~(0xFFu << sh)) | (static_cast<std::uint32_t>(pv[base + sc]) << sh);
                done |= 1u << i;
            }
        }
        const std::size_t pix = static_cast<std::size_t>(env) * 240 * 256 + y * 256 + x0;
        if (a.palette) *reinterpret_cast<uint2*>(a.palette + pix) = make_uint2(out[0], out[1]);
        if (a.rgb) {
            std::uint32_t w[6] = {0, 0, 0, 0, 0, 0};
            for (std::uint32_t i = 0; i < 8; ++i) {
                const std::uint32_t c = byte_of(out, i);
                for (std::uint32_t ch = 0; ch < 3; ++ch) {
                    const std::uint32_t b = 3 * i + ch;
                    w[b >> 2] |= static_cast<std::uint32_t>(tab.rgb[3 * c + ch]) << (8 * (b & 3));
                }
            }
            uint2* o = reinterpret_cast<uint2*>(a.rgb + pix * 3);
            o[0] = make_uint2(w[0], w[1]);
            o[1] = make_uint2(w[2], w[3]);
            o[2] = make_uint2(w[4], w[5]);
        }
        if (a.gray) {
            std::uint32_t g[2] = {0, 0};
            for (std::uint32_t i = 0; i < 8; ++i) g[i >> 2] |= static_cast<std::uint32_t>(tab.gray[byte_of(out, i)]) << (8 * (i & 3));
            *reinterpret_cast<uint2*>(&gband[r][x0]) = make_uint2(g[0], g[1]);
        }
        __syncthreads();
        if (a.gray && h_rows != 0) {   // horizontal pass of the band: column h_ox of rows h_r0, +3, +6
            for (std::uint32_t rr = h_r0; rr < kBand; rr += 3) {
                std::int32_t acc = 1 << (render::kPrecision - 1);
                for (std::uint32_t j = 0; j < render::kHTaps; ++j) acc += gband[rr][h_lo + j] * h_k[j];
                mid[(y0 + rr) % kRing][h_ox] = static_cast<std::uint8_t>(clip8(acc));
            }
        }
        __syncthreads();
        if (a.gray) {   // vertical pass of every output row whose window is now complete
            std::uint32_t end = next_oy;
            while (end < render::kOut && static_cast<std::uint32_t>(tab.taps.v_lo[end] + tab.taps.v_n[end]) <= y0 + kBand)
                ++end;
            std::uint8_t* out = a.gray + static_cast<std::size_t>(env) * render::kOut * render::kOut;
            for (std::uint32_t i = next_oy * render::kOut + tid; i < end * render::kOut; i += kThreads) {
                const std::uint32_t oy = i / render::kOut, ox = i % render::kOut;
                std::int32_t acc = 1 << (render::kPrecision - 1);
                const std::uint32_t lo = tab.taps.v_lo[oy], n = tab.taps.v_n[oy];
                for (std::uint32_t j = 0; j < n; ++j) acc += mid[(lo + j) % kRing][ox] * tab.taps.v_k[oy][j];
                out[i] = static_cast<std::uint8_t>(clip8(acc));
            }
            next_oy = end;
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

Tables make_tables() {
    Tables t{};
    axis<kHTaps>(256, t.taps.h_lo, t.taps.h_n, t.taps.h_k);
    axis<kVTaps>(240, t.taps.v_lo, t.taps.v_n, t.taps.v_k);
    // numpy's float luma of the RGB frame (an FMA chain over the channels),
    // truncated to uint8.
    for (std::uint32_t c = 0; c < 64; ++c) {
        const double r = kNesRgbHost[3 * c], g = kNesRgbHost[3 * c + 1], b = kNesRgbHost[3 * c + 2];
        t.gray[c] = static_cast<std::uint8_t>(static_cast<int>(std::fma(b, 0.114, std::fma(g, 0.587, r * 0.299))));
    }
    for (std::uint32_t i = 0; i < 192; ++i) t.rgb[i] = kNesRgbHost[i];
    return t;
}

}  // namespace render

hipError_t launch_render(const RenderArgs& a, hipStream_t stream) {
    if (a.n == 0) return hipSuccess;
    render_kernel<<<dim3(a.n), dim3(kThreads), 0, stream>>>(a);
    return hipGetLastError();
}

}  // namespace nesle
