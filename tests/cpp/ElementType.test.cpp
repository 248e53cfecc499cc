// The two-byte cache element types of paged_attention_decode<T>: bf16 and the
// IEEE binary16 f16. f16's conversions are checked against the x86 F16C
// instructions (vcvtps2ph with round-to-nearest-even, vcvtph2ps) on every
// half bit pattern and on a stride through every float exponent and
// mantissa, plus the rounding boundaries written out by hand; bf16 against
// its closed forms.
#include "minitest.h"
#include "qwenvl_paged/PagedAttention.h"

#include <immintrin.h>

#include <cmath>
#include <cstdint>
#include <cstring>

using namespace qwenvl_paged;

namespace {

float from_bits(std::uint32_t u) {
    float f;
    std::memcpy(&f, &u, sizeof f);
    return f;
}

std::uint32_t bits_of(float f) {
    std::uint32_t u;
    std::memcpy(&u, &f, sizeof u);
    return u;
}

__attribute__((target("f16c"))) std::uint16_t hw_half(float f) {
    return static_cast<std::uint16_t>(_cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC));
}

__attribute__((target("f16c"))) float hw_float(std::uint16_t h) { return _cvtsh_ss(h); }

bool have_f16c() { return __builtin_cpu_supports("f16c"); }

}  // namespace

TEST(ElementTypeTest, F16ToFloatMatchesF16cOnEveryPattern) {
    if (!have_f16c()) return;
    for (std::uint32_t h = 0; h < 65536; ++h) {
        f16 x;
        x.bits = static_cast<std::uint16_t>(h);
        const float got = float(x);
        const float want = hw_float(static_cast<std::uint16_t>(h));
        if (std::isnan(want)) {
            ASSERT_TRUE(std::isnan(got)) << "pattern " << h;
        } else {
            ASSERT_EQ(bits_of(got), bits_of(want)) << "pattern " << h;
        }
    }
}

TEST(ElementTypeTest, FloatToF16MatchesF16cAcrossTheFloatRange) {
    if (!have_f16c()) return;
    // Every exponent, both signs, mantissas on a stride that also lands on
    // the patterns next to the rounding points (low 13 bits 0x0fff..0x1001).
    for (std::uint64_t u = 0; u <= 0xffffffffull; u += 4093) {
        const float f = from_bits(static_cast<std::uint32_t>(u));
        const std::uint16_t want = hw_half(f);
        const std::uint16_t got = f16(f).bits;
        if (std::isnan(f)) {
            ASSERT_EQ(got & 0x7c00u, 0x7c00u) << "NaN in " << u;
            ASSERT_NE(got & 0x3ffu, 0u) << "NaN in " << u;
        } else {
            ASSERT_EQ(got, want) << "float bits " << u;
        }
    }
    // Every value halfway between two halves and its neighbours.
    for (std::uint32_t h = 0; h < 0x7c00u; ++h) {
        f16 lo;
        lo.bits = static_cast<std::uint16_t>(h);
        f16 hi;
        hi.bits = static_cast<std::uint16_t>(h + 1);
        const double mid = (double(float(lo)) + double(float(hi))) / 2.0;
        const float m = static_cast<float>(mid);  // exact: halves have 11 significant bits
        for (std::uint32_t v : {bits_of(m) - 1, bits_of(m), bits_of(m) + 1}) {
            for (std::uint32_t sign : {0u, 0x80000000u}) {
                const float f = from_bits(v | sign);
                ASSERT_EQ(f16(f).bits, hw_half(f)) << "near the midpoint above pattern " << h;
            }
        }
    }
}

TEST(ElementTypeTest, F16RoundingBoundaries) {
    EXPECT_EQ(f16(1.0f).bits, 0x3c00u);
    EXPECT_EQ(f16(-0.0f).bits, 0x8000u);
    EXPECT_EQ(f16(65504.0f).bits, 0x7bffu);
    EXPECT_EQ(f16(65519.996f).bits, 0x7bffu);
    EXPECT_EQ(f16(65520.0f).bits, 0x7c00u) << "halfway to 2^16 rounds to even: infinity";
    EXPECT_EQ(f16(std::ldexp(1.0f, -14)).bits, 0x0400u) << "smallest normal";
    EXPECT_EQ(f16(std::ldexp(1.0f, -24)).bits, 0x0001u) << "smallest subnormal";
    EXPECT_EQ(f16(std::ldexp(1.0f, -25)).bits, 0x0000u) << "halfway to the smallest subnormal: even is zero";
    EXPECT_EQ(f16(std::ldexp(3.0f, -25)).bits, 0x0002u) << "1.5 units of 2^-24 rounds to 2";
    EXPECT_EQ(f16(std::ldexp(1023.5f, -24)).bits, 0x0400u) << "rounds up out of the subnormals";
    EXPECT_EQ(f16(1.0f + std::ldexp(1.0f, -11)).bits, 0x3c00u) << "tie to even";
    EXPECT_EQ(f16(1.0f + std::ldexp(3.0f, -11)).bits, 0x3c02u) << "tie to even";
    EXPECT_TRUE(std::isnan(float(f16(std::nanf("")))));
    EXPECT_TRUE(std::isinf(float(f16(1e30f))));
}

TEST(ElementTypeTest, Bf16RoundsToNearestEven) {
    EXPECT_EQ(bf16(1.0f).bits, 0x3f80u);
    EXPECT_EQ(bf16(from_bits(0x3f808000u)).bits, 0x3f80u) << "tie to even (down)";
    EXPECT_EQ(bf16(from_bits(0x3f818000u)).bits, 0x3f82u) << "tie to even (up)";
    EXPECT_EQ(bf16(from_bits(0x3f808001u)).bits, 0x3f81u);
    EXPECT_EQ(bf16(from_bits(0x7f7fffffu)).bits, 0x7f80u) << "largest float rounds to infinity";
    EXPECT_TRUE(std::isnan(float(bf16(std::nanf("")))));
    for (std::uint32_t h = 0; h < 65536; ++h) {
        bf16 x;
        x.bits = static_cast<std::uint16_t>(h);
        const float f = float(x);
        ASSERT_EQ(bits_of(f), h << 16);
        if (!std::isnan(f)) {
            ASSERT_EQ(bf16(f).bits, h);
        }
    }
}
