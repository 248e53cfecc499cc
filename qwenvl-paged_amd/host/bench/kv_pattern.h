#pragma once
// Seeded synthetic contents for verifying drivers: every K/V row and query row
// is a function of its coordinates only, so a check can recompute what a frame
// must hold (or what a query was) from the sequence id and token position,
// whichever frames, swap slots or batch rows the bytes went through.
//
// Row key: k = mix(seq * G + 2 * pos + stream + C_KV) for K (stream 0) and V
// (stream 1); q = mix(row * G2 + C_Q) for the query row of batch position
// `row`. Element e of a row takes 16 bits of mix(key + (e / 4 + 1) * G),
// chunk e % 4 counted from the low end, turned into a bf16 value:
// sign = bit 15, mantissa = bits 0..6, exponent = base + (bits 7..14) % 3
// (base 124 for K/V: magnitudes in [1/16, 1); 125 for queries: [1/8, 2)).
// tests/test_gpu_configs.py restates the same function in numpy.

#include <cstddef>
#include <cstdint>

namespace kv_pattern {

constexpr std::uint64_t kGolden = 0x9E3779B97F4A7C15ull;
constexpr std::uint64_t kGolden2 = 0xD1B54A32D192ED03ull;
constexpr std::uint64_t kKvSalt = 0x632BE59BD9B4E019ull;
constexpr std::uint64_t kQuerySalt = 0x8CB92BA72F3D8DD7ull;

inline std::uint64_t mix(std::uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline std::uint16_t to_bf16(std::uint32_t chunk, std::uint32_t exponent_base) {
    const std::uint32_t exponent = exponent_base + ((chunk >> 7) & 0xFFu) % 3u;
    return static_cast<std::uint16_t>((chunk & 0x8000u) | (exponent << 7) | (chunk & 0x7Fu));
}

// n bf16 elements (n a multiple of 4) of the row with key `key`.
inline void fill_row(std::uint64_t key, std::uint32_t exponent_base, std::uint16_t* out, std::size_t n) {
    for (std::size_t g = 0; g < n / 4; ++g) {
        const std::uint64_t x = mix(key + (g + 1) * kGolden);
        for (int c = 0; c < 4; ++c) out[4 * g + c] = to_bf16(static_cast<std::uint32_t>(x >> (16 * c)) & 0xFFFFu, exponent_base);
    }
}

inline std::uint64_t kv_key(std::uint64_t seq, std::uint64_t pos, std::uint32_t stream) {
    return mix(seq * kGolden + 2 * pos + stream + kKvSalt);
}

inline std::uint64_t query_key(std::uint64_t row) { return mix(row * kGolden2 + kQuerySalt); }

// K (stream 0) or V (stream 1) row of token `pos` of sequence `seq`:
// n = num_kv_heads * head_dim elements, kv head major.
inline void kv_row(std::uint64_t seq, std::uint64_t pos, std::uint32_t stream, std::uint16_t* out, std::size_t n) {
    fill_row(kv_key(seq, pos, stream), 124, out, n);
}

// Query row of batch position `row`: n = num_query_heads * head_dim elements.
inline void query_row(std::uint64_t row, std::uint16_t* out, std::size_t n) { fill_row(query_key(row), 125, out, n); }

}  // namespace kv_pattern
