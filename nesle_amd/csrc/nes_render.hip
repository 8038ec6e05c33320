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
// RGB uses the renderer's 64-entry palette.  A render of live state follows
// the reference CPU core's renderer instead (ppu.hpp:213-545, what its
// Console shows): records built from the current registers and video memory,
// one scroll for the whole frame, a background pixel opaque whenever its
// pattern colour is non-zero, and CHR RAM read.  The gray observation is the
// pixel preprocessing of the reference's training project (project/
// mario-rl-ram/src/mario_rl/wrappers.py:209-215): luma truncated to 8 bits,
// then Pillow's BILINEAR resize to 84x84; the host computes its fixed-point
// weights (nes_render.h).
//
// One workgroup of 256 threads renders one console in bands of 8 rows, in
// three phases per band:
//  1. background: a thread owns 8 adjacent pixels of one row.  It reads the
//     (at most two) tiles under them -- nametable byte, attribute, both
//     pattern planes in one 16-bit read -- and turns each pixel's colour
//     index and tile into a byte selector, so that one v_perm over the two
//     tiles' palette words yields 4 display values (and one more 4 gray
//     levels);
//  2. sprites: the sprites that meet the band are compacted by a ballot, and
//     each (sprite, row) pair is one lane, which writes its opaque pixels as
//     keys (OAM index, gray level, palette value) into the band's line buffer
//     with an LDS atomic minimum -- the lowest OAM index wins, whatever the
//     order;
//  3. merge: a thread reads its 8 keys and replaces the background where a
//     sprite key is present, all by byte permutes; it writes the full-size
//     outputs as 8-byte runs (coalesced across the 32 threads of a row), and
//     the band's gray levels feed the horizontal resample pass in LDS; the
//     vertical pass runs once the intermediate rows an output row needs are
//     complete.  Both passes sum an 8-input window with 4-way byte dot
//     products over the weights' byte planes (exact), and run beside the
//     next band's phases, so a band costs two barriers.
// Pattern tables (8 KB, shared by every console) are staged in LDS per
// workgroup with the two planes of a tile row side by side, zeros for CHR RAM.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstddef>
#include <cstdint>

#include "nes_layout.h"
#include "nes_render.h"

namespace nesle {
namespace {

constexpr std::uint32_t kThreads = 256;
constexpr std::uint32_t kWaves = kThreads / 64;
constexpr std::uint32_t kBand = 8;
// Horizontally resampled rows kept for the vertical pass.  An output row is
// emitted after the first band that completes its input window; windows are
// at most 7 rows and end within the band, so no emitted row reaches back more
// than 14 rows and the next band overwrites only rows no pending output needs.
constexpr std::uint32_t kRing = 16;
constexpr std::uint32_t kMidStride = 2 * kRing + 4;
constexpr std::uint32_t kGrayStride = 256 + 8;
// Empty line-buffer entry; a sprite key is (OAM index << 16) | (gray << 8) |
// palette value, always below it (bit 31 clear, value byte <= 0x3F).
constexpr std::uint32_t kNoSprite = 0xFFFFFFFFu;
// The tables are staged in 16-byte words and a row of vertical weights is
// read as two of them.
static_assert(offsetof(render::Tables, s) % 16 == 0 && sizeof(render::Staged) % 16 == 0, "tables staged in 16-byte words");
static_assert(offsetof(render::Staged, v.kb) % 16 == 0, "vertical weights: two 16-byte reads per row");
// LDS of one workgroup, the sum of the kernel's shared arrays.  LDS is
// allocated in 1,280-byte units: 32,000 bytes (25 units) lets 5 workgroups
// share a compute unit's 160 KiB; one unit more leaves room for 4, and the
// kernel runs about 14 % slower.
constexpr std::size_t kLdsBytes = 2 * 4096 + present::kMaxBytes + 4 * kBand * 256 + 2 * kBand * kGrayStride +
                                  render::kOut * kMidStride + sizeof(render::Staged) + 2 * 4 * sizeof(uint2) +
                                  4 * sizeof(std::uint32_t) + kWaves * 64;
static_assert(kLdsBytes <= 32000, "render kernel LDS above 25 allocation units: 4 workgroups per compute unit");

// Scroll/ctrl pair one part of the frame is drawn with.
struct View {
    std::uint32_t ctrl, sx, sy;
};

// v_perm_b32: byte i of the result is byte sel_i of the 8-byte value hi:lo
// (0-3 lo, 4-7 hi; 8-11 replicate the sign bit of byte 1/3 of lo / hi; 12 zero).
__device__ __forceinline__ std::uint32_t perm(std::uint32_t hi, std::uint32_t lo, std::uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}
// Bits 0-3 of n to bit 0 of bytes 0-3 (the four partial products do not overlap).
__device__ __forceinline__ std::uint32_t spread4(std::uint32_t n) { return __umul24(n & 15u, 0x00204081u) & 0x01010101u; }
// Byte selectors of 4 pixels: colour index from plane bits lo/hi (bits 0-3)
// plus 4 where bit t is set (the second of two palette words).
__device__ __forceinline__ std::uint32_t selectors(std::uint32_t lo, std::uint32_t hi, std::uint32_t t) {
    return spread4(lo) | (spread4(hi) << 1) | (spread4(t) << 2);
}

// The two tiles under an 8-pixel window: pattern planes of the tile pair,
// pixel p (0..15, left to right) at bit p (low plane) and bit 16 + p (high
// plane); both tiles' attribute palettes; the window's offset into the pair.
struct TilePair {
    std::uint32_t planes, pal0, pal1, fx;
};

struct Console {
    const std::uint16_t* chr;   // LDS, pattern table rows: low plane | high plane << 8
    const std::uint8_t* nt;     // LDS, snapshot nametable RAM
    std::uint32_t mask;
    // Nametable n = x | y << 1 lives at (x * mx + y * my) * 0x400 of nametable
    // RAM: vertical mirroring mx = 1, my = 0; horizontal 0, 1; four-screen 1, 2.
    std::uint32_t mx, my;

    // batch_background_color (batch_render.cuh:219-262) for the window
    // x..x+7 of row y: the frame is a 512 x 480 world of 2 x 2 nametables,
    // scrolled by (sx, sy) from the nametable ctrl selects, rows wrapping at 480.
    __device__ TilePair tiles(const View& w, std::uint32_t x, std::uint32_t y) const {
        std::uint32_t wy = w.sy + y + ((w.ctrl & 2) ? 240u : 0u);
        if (wy >= 480) wy -= 480;
        const std::uint32_t ty = wy >> 3, fine_y = wy & 7;
        const bool lower = ty >= 30;
        const std::uint32_t cy = lower ? ty - 30 : ty;
        const std::uint32_t row = (lower ? my << 10 : 0u) + cy * 32;
        const std::uint32_t arow = (lower ? my << 10 : 0u) + 0x3C0 + (cy >> 2) * 8;
        const std::uint32_t ashift = (cy & 2) << 1;
        const std::uint32_t wx = w.sx + x + ((w.ctrl & 1) ? 256u : 0u);
        const std::uint32_t pt = (w.ctrl & 0x10) ? 256u : 0u;
        std::uint32_t pat[2], pal[2];
        for (std::uint32_t k = 0; k < 2; ++k) {
            const std::uint32_t tx = ((wx >> 3) + k) & 63, cx = tx & 31;
            const std::uint32_t ntx = (tx & 32) ? mx << 10 : 0u;
            const std::uint32_t tile = nt[row + ntx + cx];
            const std::uint32_t attr = nt[arow + ntx + (cx >> 2)];
            pal[k] = (attr >> (ashift | (cx & 2))) & 3;
            pat[k] = chr[(pt + tile) * 8 + fine_y];
        }
        // Bit-reverse the word [lo0, hi0, lo1, hi1] to [rhi1, rlo1, rhi0, rlo0]
        // and reorder to [rlo0, rlo1, rhi0, rhi1]: leftmost pixel at bit 0.
        const std::uint32_t r = __builtin_bitreverse32(pat[0] | (pat[1] << 16));
        return {perm(r, r, 0x00020103u), pal[0], pal[1], wx & 7};
    }

    // Opacity (bit i: pixel x + i) of the background of the window x..x+7
    // of row y: colour index not 0 and palette value not 0, nothing where the
    // background is off or hidden in the left column.
    __device__ std::uint32_t opacity(const View& w, std::uint32_t x, std::uint32_t y, const std::uint32_t* bgo) const {
        if (!(mask & 0x08)) return 0;
        const TilePair p = tiles(w, x, y);
        const std::uint32_t lo = p.planes >> p.fx, hi = p.planes >> (p.fx + 16), t = 0xFF00u >> p.fx;
        const std::uint32_t a = bgo[p.pal0], b = bgo[p.pal1];
        // Opacity bytes (0 or 1) of pixels 0-3 and 4-7, gathered to 4 bits each.
        const std::uint32_t o0 = perm(b, a, selectors(lo, hi, t)) * 0x01020408u >> 24;
        const std::uint32_t o1 = perm(b, a, selectors(lo >> 4, hi >> 4, t >> 4)) * 0x01020408u >> 24;
        std::uint32_t o = o0 | (o1 << 4);
        if (!(mask & 0x02) && x < 8) o &= (0xFF00u >> x) & 0xFFu;
        return o;
    }
};

__device__ __forceinline__ std::uint32_t byte_of(const std::uint32_t w[2], std::uint32_t i) {
    return (w[i >> 2] >> (8 * (i & 3))) & 0xFF;
}

// Bytes p..p+7 of a 4-byte-aligned LDS row (p & ~3 plus 11 inside it): three
// aligned dword reads and two byte funnel shifts (an unaligned 8-byte LDS
// read costs the LDS pipeline several passes).
__device__ __forceinline__ uint2 bytes8(const std::uint8_t* row, std::uint32_t p) {
    const std::uint32_t* d = reinterpret_cast<const std::uint32_t*>(row + (p & ~3u));
    const std::uint32_t d0 = d[0], d1 = d[1], d2 = d[2];
    return make_uint2(__builtin_amdgcn_alignbyte(d1, d0, p & 3), __builtin_amdgcn_alignbyte(d2, d1, p & 3));
}

// Pillow's fixed-point sum of 8 consecutive 8-bit inputs (bytes of w) with
// weights given as byte planes (pack_weights), rounded: three pairs of
// 4-way byte dot products.
__device__ __forceinline__ std::int32_t window8(const uint2 w, const std::uint32_t kb[6]) {
    std::uint32_t d[3];
    for (std::uint32_t b = 0; b < 3; ++b)
        d[b] = __builtin_amdgcn_udot4(w.y, kb[3 + b], __builtin_amdgcn_udot4(w.x, kb[b], 0u, false), false);
    return static_cast<std::int32_t>((1u << (render::kPrecision - 1)) + d[0] + (d[1] << 8) + (d[2] << 16));
}

__device__ __forceinline__ std::uint32_t clip8(std::int32_t acc) {
    const std::int32_t v = acc >> render::kPrecision;
    return static_cast<std::uint32_t>(v < 0 ? 0 : (v > 255 ? 255 : v));
}

// Sprite pixels of 4 line-buffer keys over background words: display
// values d and gray levels g of the 4 pixels, background where no key.
__device__ __forceinline__ void merge(const uint4 k, std::uint32_t& d, std::uint32_t& g) {
    const std::uint32_t t = perm(k.y, k.x, 0x05010400u);        // [v0, v1, g0, g1]
    const std::uint32_t u = perm(k.w, k.z, 0x05010400u);        // [v2, v3, g2, g3]
    const std::uint32_t v = perm(u, t, 0x05040100u);            // values
    const std::uint32_t gr = perm(u, t, 0x07060302u);           // gray levels
    // 0xFF where the value byte is 0xFF (no key), from the bytes' sign bits.
    const std::uint32_t none = perm(v << 8, v, 0x090B080Au);
    d = (none & d) | (~none & v);
    g = (none & g) | (~none & gr);
}

__global__ void __launch_bounds__(kThreads) render_kernel(RenderArgs a) {
    __shared__ __attribute__((aligned(16))) std::uint16_t chr[4096];          // [512 tiles][8 rows]
    __shared__ __attribute__((aligned(16))) std::uint8_t rec[present::kMaxBytes];
    __shared__ __attribute__((aligned(16))) std::uint32_t line[kBand][256];   // sprite keys of the band
    // Gray rows of the last two bands (rows padded so a window's third dword
    // stays inside its row).
    __shared__ __attribute__((aligned(16))) std::uint8_t gband[2][kBand][kGrayStride];
    // Horizontally resampled rows, column-major, the ring stored twice so an
    // output's window (kWindow rows from any ring position) is contiguous; a
    // column takes 9 dwords, so the 64 columns a wave touches fall in
    // distinct LDS banks.
    __shared__ __attribute__((aligned(16))) std::uint8_t mid[render::kOut][kMidStride];
    __shared__ __attribute__((aligned(16))) render::Staged tab;
    __shared__ uint2 bgw[4];          // background palettes: display values, gray levels
    __shared__ uint2 spw[4];          // sprite palettes: palette values, gray levels
    __shared__ std::uint32_t bgo[4];  // background palettes: 1 where opaque
    __shared__ std::uint8_t list[kWaves][64];   // per wave: sprites that meet the band

    const std::uint32_t tid = threadIdx.x, env = blockIdx.x;
    {
        const uint4* src = reinterpret_cast<const uint4*>(a.present + static_cast<std::size_t>(env) * a.present_stride);
        for (std::uint32_t i = tid; i < a.present_stride / 16; i += kThreads) reinterpret_cast<uint4*>(rec)[i] = src[i];
        // Pattern tables: the CHR ROM (an image smaller than 8 KB repeats), or
        // zeros for CHR RAM, which the batched renderer reads as 0.  A tile's
        // 16 bytes (8 low-plane rows, 8 high-plane rows) become 8 row pairs.
        const std::uint32_t words = a.chr_size / 16;
        const uint4* c = reinterpret_cast<const uint4*>(a.chr);
        // CHR RAM under the CPU core's rules: this console's bytes, gathered
        // from the interleaved rows (byte `addr` of console env at addr * pitch + env).
        const std::uint8_t* cram = (a.cpu_rules != 0 && words == 0) ? a.chr_ram : nullptr;
        for (std::uint32_t i = tid; i < 512; i += kThreads) {
            uint4 t = words != 0 ? c[i % words] : make_uint4(0, 0, 0, 0);
            if (cram != nullptr) {
                std::uint32_t w[4];
                for (std::uint32_t q = 0; q < 4; ++q) {
                    w[q] = 0;
                    for (std::uint32_t j = 0; j < 4; ++j)
                        w[q] |= static_cast<std::uint32_t>(cram[static_cast<std::size_t>(16 * i + 4 * q + j) * a.pitch + env]) << (8 * j);
                }
                t = make_uint4(w[0], w[1], w[2], w[3]);
            }
            reinterpret_cast<uint4*>(chr)[i] = make_uint4(perm(t.z, t.x, 0x05010400u), perm(t.z, t.x, 0x07030602u),
                                                          perm(t.w, t.y, 0x05010400u), perm(t.w, t.y, 0x07030602u));
        }
        const uint4* t = reinterpret_cast<const uint4*>(&a.tables->s);
        for (std::uint32_t i = tid; i < sizeof(render::Staged) / 16; i += kThreads) reinterpret_cast<uint4*>(&tab)[i] = t[i];
        for (std::uint32_t i = tid; i < kBand * 256 / 4; i += kThreads)
            reinterpret_cast<uint4*>(line)[i] = make_uint4(kNoSprite, kNoSprite, kNoSprite, kNoSprite);
    }
    __syncthreads();

    const std::uint32_t mask = rec[present::kMask];
    const std::uint8_t* oam = rec + present::kOam;
    if (tid < 8) {
        // batch_palette_value: aliases of $3F10/14/18/1C, grayscale, 6 bits.
        auto value = [&](std::uint32_t i) {
            std::uint32_t v = rec[present::kPalette + (((i & 0x13) == 0x10) ? (i & 0x0F) : i)];
            if (mask & 0x01) v &= 0x30;
            return v & 0x3F;
        };
        const std::uint32_t q = tid & 3;
        std::uint32_t v = 0, g = 0, o = 0;
        for (std::uint32_t c = 0; c < 4; ++c) {
            std::uint32_t p;
            if (tid < 4) {   // background: colour 0 (and, batched rules, value 0) shows the backdrop, transparent
                p = value(4 * q + c);
                const bool opaque = c != 0 && (p != 0 || a.cpu_rules != 0);
                if (!opaque) p = value(0);
                o |= (opaque ? 1u : 0u) << (8 * c);
            } else {
                p = value(16 + 4 * q + c);
            }
            v |= p << (8 * c);
            g |= static_cast<std::uint32_t>(a.tables->gray[p]) << (8 * c);
        }
        if (tid < 4) {
            bgw[q] = make_uint2(v, g);
            bgo[q] = o;
        } else {
            spw[q] = make_uint2(v, g);
        }
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
    __syncthreads();

    const Console con{chr, rec + present::kNametable, mask, a.nt_mode == 1 ? 0u : 1u,
                      a.nt_mode == 2 ? 2u : a.nt_mode == 1 ? 1u : 0u};
    const std::uint32_t r = tid >> 5, x0 = (tid & 31) * 8;
    const std::uint32_t lane = tid & 63, wave = tid >> 6;
    const std::uint32_t backdrop = bgw[0].x & 0xFF, backdrop_gray = bgw[0].y & 0xFF;
    const bool bg_on = (mask & 0x08) && (x0 != 0 || (mask & 0x02));   // else this run shows the backdrop
    const bool clip = !(mask & 0x04);                                  // sprites hidden in the left column
    std::uint32_t next_oy = 0;   // first gray row not yet written
    // Resample passes: thread t < 252 owns output column t % 84, for band rows
    // t / 84, +3, +6 of the horizontal pass and output rows t / 84, +3, ... of
    // the vertical pass.  The column's horizontal weights sit in registers,
    // over the 8 inputs from h_lo (taps past the window's end weigh 0 and
    // read inside the row).
    const std::uint32_t h_rows = tid < 3 * render::kOut ? 1u : 0u;
    const std::uint32_t h_ox = tid % render::kOut, h_r0 = tid / render::kOut;
    std::int32_t h_w[render::kWindow];
    const render::Axis<render::kHTaps>& ht = a.tables->h;
    const std::int32_t first = ht.lo[h_ox], taps = ht.n[h_ox];
    const std::uint32_t h_lo = first + render::kWindow > 256 ? 256 - render::kWindow : first;
    for (std::uint32_t j = 0; j < render::kWindow; ++j) {
        const std::int32_t k = static_cast<std::int32_t>(j + h_lo) - first;   // tap index of input h_lo + j
        h_w[j] = (k >= 0 && k < taps) ? ht.k[h_ox][k] : 0;
    }
    std::uint32_t h_k[6];
    render::pack_weights(h_w, h_k);
    // Band k is drawn in iteration k (background and sprites, then the merge)
    // while iteration k + 1 resamples it (horizontal pass beside band k + 1's
    // background and sprites, vertical pass beside its merge): two barriers a
    // band.  The gray rows of a band alternate between two buffers.
    constexpr std::uint32_t kBands = 240 / kBand;
    for (std::uint32_t band = 0; band <= kBands; ++band) {
        const bool draw = band < kBands, resample = a.gray && band > 0;
        const std::uint32_t y0 = band * kBand, y = y0 + r;
        std::uint32_t d[2], g[2];
        if (draw) {
            // 1. Background of the run: display values d (palette value 0 shows
            // the backdrop) and their gray levels g.
            d[0] = d[1] = backdrop * 0x01010101u;
            g[0] = g[1] = backdrop_gray * 0x01010101u;
            if (bg_on) {
                const TilePair p = con.tiles(static_cast<std::int32_t>(y) < split ? hud : play, x0, y);
                const std::uint32_t lo = p.planes >> p.fx, hi = p.planes >> (p.fx + 16), t = 0xFF00u >> p.fx;
                const uint2 w0 = bgw[p.pal0], w1 = bgw[p.pal1];
                for (std::uint32_t h = 0; h < 2; ++h) {
                    const std::uint32_t sel = selectors(lo >> (4 * h), hi >> (4 * h), t >> (4 * h));
                    d[h] = perm(w1.x, w0.x, sel);
                    g[h] = perm(w1.y, w0.y, sel);
                }
            }
            // 2. Sprites (batch_render.cuh:264-330) into the line buffer.
            if (mask & 0x10) {
                // Sprite `lane` covers rows oam[4 * lane] + 1 .. + height; the
                // sprites meeting rows y0..y0+7, in OAM order, to this wave's list.
                const std::uint32_t top = oam[4 * lane];
                const bool meets = top + height - y0 < height + kBand - 1;
                const std::uint64_t ball = __ballot(meets);
                const std::uint32_t count = static_cast<std::uint32_t>(__popcll(ball));
                if (meets)
                    list[wave][__builtin_amdgcn_mbcnt_hi(static_cast<std::uint32_t>(ball >> 32),
                                                         __builtin_amdgcn_mbcnt_lo(static_cast<std::uint32_t>(ball), 0u))] =
                        static_cast<std::uint8_t>(lane);
                __builtin_amdgcn_wave_barrier();
                for (std::uint32_t slot = tid; slot < count * kBand; slot += kThreads) {
                    const std::uint32_t s = list[wave][slot / kBand], row = slot % kBand, sy = y0 + row;
                    const std::uint32_t o = *reinterpret_cast<const std::uint32_t*>(oam + 4 * s);
                    const std::uint32_t attr = (o >> 16) & 0xFF, tile = (o >> 8) & 0xFF, sx = o >> 24;
                    std::uint32_t py = sy - ((o & 0xFF) + 1);
                    if (py >= height) continue;
                    std::uint32_t t;   // pattern tile 0..511
                    if (height == 16) {
                        if (attr & 0x80) py = 15 - py;
                        t = ((tile & 1) << 8) + (((tile & 0xFE) + (py >> 3)) & 0xFF);
                    } else {
                        if (attr & 0x80) py = 7 - py;
                        t = ((play.ctrl & 0x08) ? 256u : 0u) + tile;
                    }
                    std::uint32_t pat = chr[t * 8 + (py & 7)];
                    if (!(attr & 0x40)) {   // not flipped: leftmost pixel to bit 0
                        const std::uint32_t rv = __builtin_bitreverse32(pat);
                        pat = perm(rv, rv, 0x0C0C0203u);
                    }
                    std::uint32_t op = (pat | (pat >> 8)) & 0xFF;   // bit j: column j opaque
                    if (sx > 248) op &= 0xFFu >> (sx - 248);         // off the right edge
                    if (clip && sx < 8) op &= (0xFF00u >> sx) & 0xFFu;
                    if ((attr & 0x20) && op != 0) op &= ~con.opacity(play, sx, sy, bgo);   // behind the background
                    if (op == 0) continue;
                    const uint2 sp = spw[attr & 3];
                    std::uint32_t* dst = &line[row][sx];
                    for (std::uint32_t h = 0; h < 2; ++h) {
                        const std::uint32_t sel = selectors(pat >> (4 * h), pat >> (8 + 4 * h), 0);
                        for (std::uint32_t q = 0; q < 2; ++q) {
                            // (value, gray) of columns 4h + 2q and 4h + 2q + 1.
                            const std::uint32_t pair = perm(sp.y, sp.x, perm(sel, sel, 0x01010000u + 0x02020202u * q) + 0x04000400u);
                            const std::uint32_t j = 4 * h + 2 * q;
                            if ((op >> j) & 1) atomicMin(dst + j, (s << 16) | (pair & 0xFFFF));
                            if ((op >> (j + 1)) & 1) atomicMin(dst + j + 1, (s << 16) | (pair >> 16));
                        }
                    }
                }
            }
        }
        if (resample && h_rows != 0) {   // horizontal pass of the previous band: column h_ox of rows h_r0, +3, +6
            for (std::uint32_t rr = h_r0; rr < kBand; rr += 3) {
                const uint2 w = bytes8(gband[(band - 1) & 1][rr], h_lo);
                const std::uint32_t slot = (y0 - kBand + rr) % kRing;
                mid[h_ox][slot] = mid[h_ox][slot + kRing] = static_cast<std::uint8_t>(clip8(window8(w, h_k)));
            }
        }
        __syncthreads();
        if (draw) {
            // 3. Merge the run's sprite keys; the buffer is left empty for the next band.
            {
                uint4* keys = reinterpret_cast<uint4*>(&line[r][x0]);
                merge(keys[0], d[0], g[0]);
                merge(keys[1], d[1], g[1]);
                keys[0] = keys[1] = make_uint4(kNoSprite, kNoSprite, kNoSprite, kNoSprite);
            }
            const std::size_t pix = static_cast<std::size_t>(env) * 240 * 256 + y * 256 + x0;
            if (a.palette) *reinterpret_cast<uint2*>(a.palette + pix) = make_uint2(d[0], d[1]);
            if (a.rgb) {   // 8 pixels' RGB: one palette word per pixel, packed by 3 permutes per 4 pixels
                std::uint32_t c[8], w[6];
                for (std::uint32_t i = 0; i < 8; ++i) c[i] = tab.rgb[byte_of(d, i)];
                for (std::uint32_t h = 0; h < 2; ++h) {
                    const std::uint32_t* q = c + 4 * h;
                    w[3 * h] = perm(q[1], q[0], 0x04020100u);       // R0 G0 B0 R1
                    w[3 * h + 1] = perm(q[2], q[1], 0x05040201u);   // G1 B1 R2 G2
                    w[3 * h + 2] = perm(q[3], q[2], 0x06050402u);   // B2 R3 G3 B3
                }
                uint2* o = reinterpret_cast<uint2*>(a.rgb + pix * 3);
                o[0] = make_uint2(w[0], w[1]);
                o[1] = make_uint2(w[2], w[3]);
                o[2] = make_uint2(w[4], w[5]);
            }
            if (a.gray) *reinterpret_cast<uint2*>(&gband[band & 1][r][x0]) = make_uint2(g[0], g[1]);
        }
        if (resample) {   // vertical pass of every output row whose window the previous band completed
            std::uint32_t end = next_oy;
            while (end < render::kOut && static_cast<std::uint32_t>(tab.v.lo[end] + tab.v.n[end]) <= y0)
                ++end;
            std::uint8_t* out = a.gray + static_cast<std::size_t>(env) * render::kOut * render::kOut;
            for (std::uint32_t oy = next_oy + h_r0; h_rows != 0 && oy < end; oy += 3) {
                const uint2 w = bytes8(mid[h_ox], tab.v.lo[oy] % kRing);
                const uint4* k = reinterpret_cast<const uint4*>(tab.v.kb[oy]);
                const uint4 k0 = k[0], k1 = k[1];
                const std::uint32_t kv[6] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y};
                out[oy * render::kOut + h_ox] = static_cast<std::uint8_t>(clip8(window8(w, kv)));
            }
            next_oy = end;
        }
        __syncthreads();
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
    axis<kHTaps>(256, t.h.lo, t.h.n, t.h.k);
    Axis<kVTaps> v;
    axis<kVTaps>(240, v.lo, v.n, v.k);
    for (std::uint32_t oy = 0; oy < kOut; ++oy) {
        t.s.v.lo[oy] = v.lo[oy];
        t.s.v.n[oy] = v.n[oy];
        pack_weights(v.k[oy], t.s.v.kb[oy]);
    }
    // numpy's float luma of the RGB frame (an FMA chain over the channels),
    // truncated to uint8.
    for (std::uint32_t c = 0; c < 64; ++c) {
        const double r = kNesRgbHost[3 * c], g = kNesRgbHost[3 * c + 1], b = kNesRgbHost[3 * c + 2];
        t.gray[c] = static_cast<std::uint8_t>(static_cast<int>(std::fma(b, 0.114, std::fma(g, 0.587, r * 0.299))));
    }
    for (std::uint32_t c = 0; c < 64; ++c)
        t.s.rgb[c] = kNesRgbHost[3 * c] | (kNesRgbHost[3 * c + 1] << 8) | (static_cast<std::uint32_t>(kNesRgbHost[3 * c + 2]) << 16);
    return t;
}

}  // namespace render

hipError_t launch_render(const RenderArgs& a, hipStream_t stream) {
    if (a.n == 0) return hipSuccess;
    render_kernel<<<dim3(a.n), dim3(kThreads), 0, stream>>>(a);
    return hipGetLastError();
}

}  // namespace nesle
