// The float16 input activations (tanh-GELU, SiLU, SwiGLU, bit-identical to torch's CPU routines
// on float16) and the float64 -> float16 rounding of rotated values: the float16 counterparts of
// act_rot.h's pieces, for the activation-row kernels that take float16 rows.
#pragma once

#include "act_rot.h"

namespace mxq {

// ---- tanh-GELU and SiLU on float16 ---------------------------------------------------------
// Bit-exact torch CPU gelu(approximate="tanh") and silu on a float16 input (the reference applies
// them in the activation's own dtype, CK/backends/_activations.py:47-52): rules and tables from
// gen_act_f16_tables.py, which checks them against all 65,536 torch outputs of each. Biased
// exponent e (5 bits): below E_LO x / 2 with ties resolved upwards, at or above E_POS (x > 0)
// x itself, at or above E_NEG (x < 0) -0.0, e = 31 the infinities and NaNs, the rest tabled.
#define MXQ_GELU16_TABLE_DECL constexpr uint16_t kGelu16TableC[MXQ_GELU16_TABLE_SIZE]
#define MXQ_SILU16_TABLE_DECL constexpr uint16_t kSilu16TableC[MXQ_SILU16_TABLE_SIZE]
#include "act_f16_tables.inc"
#undef MXQ_GELU16_TABLE_DECL
#undef MXQ_SILU16_TABLE_DECL

template <int kELo, int kEPos, int kENeg, bool kQuietNan, uint32_t kNan, uint32_t kNinf>
constexpr uint32_t act16_rule_c(uint32_t b, const uint16_t* table) {
  const uint32_t e = (b >> 10) & 0x1Fu, sign = b & 0x8000u, mag = b & 0x7FFFu;
  if (e < (uint32_t)kELo) return sign | (e >= 2 ? mag - 0x400u : (sign ? mag >> 1 : (mag + 1) >> 1));
  if (e == 31u) return b == 0x7C00u ? 0x7C00u : (b == 0xFC00u ? kNinf : (kQuietNan ? b | 0x200u : kNan));
  if (!sign && e >= (uint32_t)kEPos) return b;
  if (sign && e >= (uint32_t)kENeg) return 0x8000u;
  return sign ? table[(kEPos - kELo) * 1024 + (e - kELo) * 1024 + (b & 0x3FFu)] : table[(e - kELo) * 1024 + (b & 0x3FFu)];
}
struct Act16FullTable {
  uint16_t v[65536];
};
constexpr Act16FullTable make_gelu16_full() {
  Act16FullTable t{};
  for (uint32_t b = 0; b < 65536u; ++b)
    t.v[b] = (uint16_t)act16_rule_c<MXQ_GELU16_E_LO, MXQ_GELU16_E_POS, MXQ_GELU16_E_NEG, MXQ_GELU16_NAN_QUIETS_INPUT != 0,
                                    MXQ_GELU16_NAN, MXQ_GELU16_NINF>(b, kGelu16TableC);
  return t;
}
constexpr Act16FullTable make_silu16_full() {
  Act16FullTable t{};
  for (uint32_t b = 0; b < 65536u; ++b)
    t.v[b] = (uint16_t)act16_rule_c<MXQ_SILU16_E_LO, MXQ_SILU16_E_POS, MXQ_SILU16_E_NEG, MXQ_SILU16_NAN_QUIETS_INPUT != 0,
                                    MXQ_SILU16_NAN, MXQ_SILU16_NINF>(b, kSilu16TableC);
  return t;
}
static __device__ __attribute__((aligned(16))) const Act16FullTable kGelu16Full = make_gelu16_full();
static __device__ __attribute__((aligned(16))) const Act16FullTable kSilu16Full = make_silu16_full();

MXQ_DEVICE uint32_t gelu_f16(uint32_t b) { return kGelu16Full.v[b & 0xFFFFu]; }
MXQ_DEVICE uint32_t silu_f16(uint32_t b) { return kSilu16Full.v[b & 0xFFFFu]; }

// SwiGLU of one float16 pair as torch's CPU silu(gate).mul_(up): the product of two float16 is
// exact in fp32, then one RNE rounding. NaNs follow the CPU's multiply: a NaN silu(gate) passes
// through, else a NaN `up` is passed on quieted, else an invalid product (0 * inf) gives the
// CPU's default NaN, negative (0xFE00).
MXQ_DEVICE uint32_t swiglu_f16(uint32_t gate, uint32_t up) {
  const uint32_t s = silu_f16(gate);
  if ((s & 0x7FFFu) > 0x7C00u) return s;
  if ((up & 0x7FFFu) > 0x7C00u) return up | 0x200u;
  const float p = f16_to_f32(s) * f16_to_f32(up);
  return p != p ? 0xFE00u : f32_to_f16_bits(p);
}

// float64 -> float16 bits with one round-to-nearest-even rounding: the float64 is first rounded
// to float32 by round-to-odd (truncate, then set the last bit if anything was cut), which keeps
// the value's side of every float16 rounding boundary, and that float32 is rounded to float16.
MXQ_DEVICE uint32_t f64_to_f16_bits(double x) {
  float f = (float)x;
  if ((double)f != x) {
    uint32_t u = __float_as_uint(f);
    if (fabs((double)f) > fabs(x)) u -= 1u;
    f = __uint_as_float(u | 1u);
  }
  return f32_to_f16_bits(f);
}

}  // namespace mxq
