// nes_render.h -- frame rendering of the batched console (nes_render.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace nesle {
namespace render {

constexpr int kPrecision = 22;             // Pillow's 8-bit resample fixed point
constexpr std::uint32_t kOut = 84;         // gray observation is kOut x kOut
constexpr std::uint32_t kHTaps = 9;        // 256 -> 84: ceil(256 / 84) * 2 + 1
constexpr std::uint32_t kVTaps = 8;        // 240 -> 84: ceil(240 / 84) * 2 + 1 = 7, padded to 8
// Inputs an output actually reads: a BILINEAR window spans at most
// 2 * scale + 1 inputs, 7.1 across (256 / 84) and 6.7 down (240 / 84), so
// 8 consecutive inputs hold every window; the kernel reads 8 bytes per output.
constexpr std::uint32_t kWindow = 8;

// Pillow BILINEAR weights of one axis: per output column or row, first
// input, input count, weights (each in [0, 2^22]; zero past the count).
template <std::uint32_t kTaps>
struct Axis {
    std::int32_t lo[kOut], n[kOut], k[kOut][kTaps];
};

// The 8 weights of a window as byte planes for v_dot4_u32_u8: word 3 * g + b
// holds byte b of the weights of inputs 4g..4g+3.  A weight is below 2^23,
// so three planes hold it and sum_j x_j k_j = d0 + (d1 << 8) + (d2 << 16),
// d_b the byte-plane dot products, exactly.
__host__ __device__ inline void pack_weights(const std::int32_t k[kWindow], std::uint32_t out[6]) {
    for (std::uint32_t g = 0; g < 2; ++g)
        for (std::uint32_t b = 0; b < 3; ++b) {
            std::uint32_t w = 0;
            for (std::uint32_t i = 0; i < 4; ++i)
                w |= ((static_cast<std::uint32_t>(k[4 * g + i]) >> (8 * b)) & 0xFFu) << (8 * i);
            out[3 * g + b] = w;
        }
}

// Vertical pass weights as the kernel reads them: first input row, input
// count, byte planes (6 words, padded to 8 for two 16-byte reads).
struct Vertical {
    std::int32_t lo[kOut], n[kOut];
    std::uint32_t kb[kOut][8];
};

// The part of the tables the render kernel keeps in LDS.
struct Staged {
    Vertical v;              // 240 rows -> 84
    std::uint32_t rgb[64];   // the renderer's RGB palette: R | G << 8 | B << 16
};

// Everything the render kernel looks up, uploaded once per batch.
struct Tables {
    Axis<kHTaps> h;          // 256 columns -> 84, read once per thread
    Staged s;
    std::uint8_t gray[64];   // gray level of each palette colour, read once per console
};

// Host: the resize weights of Pillow's BILINEAR filter (libImaging/Resample.c
// precompute_coeffs + normalize_coeffs_8bpc), the gray level of each palette
// colour, uint8(fma(b, .114, fma(g, .587, r * .299))) -- numpy's float luma of
// the RGB frame, truncated -- and the RGB palette.
Tables make_tables();

}  // namespace render

struct RenderArgs {
    std::uint32_t n;                 // consoles
    const std::uint8_t* present;     // [n][present_stride] presentation records
    std::uint32_t present_stride;    // present::kHeader + video memory block
    const std::uint8_t* chr;         // CHR ROM (device), null for CHR RAM
    std::uint32_t chr_size;          // 0 for CHR RAM
    std::uint32_t nt_mode;           // 0 vertical, 1 horizontal, 2 four-screen
    const render::Tables* tables;    // (device)
    std::uint8_t* palette;           // [n][240][256] or null
    std::uint8_t* rgb;               // [n][240][256][3] or null
    std::uint8_t* gray;              // [n][84][84] or null
    // The reference CPU core's rules (ppu.hpp:213-545) instead of the
    // batched core's: a background pixel is opaque when its pattern colour is
    // non-zero (whatever its palette value), and CHR RAM is read.  Used with
    // records of live state (start = end, so one scroll for the frame).
    std::uint32_t cpu_rules;
    const std::uint8_t* chr_ram;     // interleaved [8192][pitch] CHR RAM, or null
    std::uint32_t pitch;
};

hipError_t launch_render(const RenderArgs& a, hipStream_t stream);

}  // namespace nesle
