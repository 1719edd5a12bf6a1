// Shared pieces of the kernels that quantize activation rows: the SiLU / SwiGLU input
// activation (bit-identical to torch's CPU routines on bfloat16), the float64 -> bfloat16
// rounding of rotated values, and the radix-4 step of the ConvRot (regular Hadamard) rotation.
#pragma once

#include "mxq_common.h"

namespace mxq {

// ---- SiLU on bfloat16 ---------------------------------------------------------------------
// Bit-exact torch CPU silu on a bfloat16 input (the gate activation of the reference's SwiGLU,
// CK/backends/_activations.py:50-52); rules and table from gen_silu_table.py, which checks them
// against all 65,536 torch outputs.
#define MXQ_SILU_TABLE_DECL constexpr uint16_t kSiluTableC[3840]
#include "silu_bf16_table.inc"
#undef MXQ_SILU_TABLE_DECL

constexpr uint32_t silu_rule_c(uint32_t b) {
  const uint32_t e = (b >> 7) & 0xFFu, sign = b & 0x8000u, mag = b & 0x7FFFu;
  if (e < MXQ_SILU_E_LO) {
    const uint32_t v = mag & 0xFFu;
    return sign | (e >= 2 ? mag - 0x80u : (v >> 1) + ((v & 1u) & ((v >> 1) & 1u)));
  }
  if (e == 255u) return b == 0x7F80u ? 0x7F80u : MXQ_SILU_NAN;
  if (!sign && e >= MXQ_SILU_E_POS) return b;
  if (sign && e >= MXQ_SILU_E_NEG) return 0x8000u;
  return kSiluTableC[((b >> 15) * (MXQ_SILU_E_NEG - MXQ_SILU_E_LO) + (e - MXQ_SILU_E_LO)) * 128u + (b & 0x7Fu)];
}
struct SiluFullTable {
  uint16_t v[65536];
};
constexpr SiluFullTable make_silu_full() {
  SiluFullTable t{};
  for (uint32_t b = 0; b < 65536u; ++b) t.v[b] = (uint16_t)silu_rule_c(b);
  return t;
}
static __device__ __attribute__((aligned(16))) const SiluFullTable kSiluFull = make_silu_full();

MXQ_DEVICE uint32_t silu_bf16(uint32_t b) { return kSiluFull.v[b & 0xFFFFu]; }

// SwiGLU of one bf16 pair: bf16(bf16(silu(gate)) * up) -- the product of two bf16 is exact in
// fp32, so this is torch's bf16 mul_ (one rounding); a NaN product becomes 0x7FC0, the pattern
// torch's float -> bfloat16 conversion gives every NaN.
MXQ_DEVICE uint32_t swiglu_bf16(uint32_t gate, uint32_t up) {
  const float p = bf16_to_f32(silu_bf16(gate)) * bf16_to_f32(up);
  return p != p ? 0x7FC0u : f32_to_bf16_bits(p);
}

// float64 -> bfloat16 bits with one round-to-nearest-even rounding: through float32 (RNE),
// exact except where that float32 is itself a bfloat16 midpoint and x is not; then x lies
// strictly on one side of the midpoint and the result is the neighbour on that side.
MXQ_DEVICE uint32_t f64_to_bf16_bits(double x) {
  const float f = (float)x;
  const uint32_t u = __float_as_uint(f);
  uint32_t b = f32_to_bf16_bits(f);
  if ((u & 0xFFFFu) == 0x8000u && (double)f != x) b = (u >> 16) + (fabs(x) > fabs((double)f) ? 1u : 0u);
  return b;
}

// One radix-4 step on four values (the quad of one digit).
// y_k = S - 2 x_{3-k} is one fma: -2 x is exact, so fma(-2, x, S) rounds S - (x + x) once, as
// the separate doubling and subtraction do.
MXQ_DEVICE void h4_quad(double& x0, double& x1, double& x2, double& x3) {
  const double s = (x0 + x1) + (x2 + x3);
  const double y0 = __builtin_fma(-2.0, x3, s), y1 = __builtin_fma(-2.0, x2, s);
  const double y2 = __builtin_fma(-2.0, x1, s), y3 = __builtin_fma(-2.0, x0, s);
  x0 = y0;
  x1 = y1;
  x2 = y2;
  x3 = y3;
}

// Loads 16 consecutive bf16 activations of one lane (columns e0 .. e0 + 15 of a row; zeros when
// !on), applies the input activation (kAct; SwiGLU reads gate at xr[e] and up at xr[K + e]) and
// returns them as float64.
template <int kAct>
MXQ_DEVICE void load16_act(const uint16_t* xr, int64_t K, int e0, bool on, double* v) {
  v4u w[2], up[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    w[c] = on ? reinterpret_cast<const v4u*>(xr + e0)[c] : v4u{0, 0, 0, 0};
    if (kAct == MXQ_ACT_SWIGLU) up[c] = on ? reinterpret_cast<const v4u*>(xr + K + e0)[c] : v4u{0, 0, 0, 0};
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t word = w[i >> 3][(i >> 1) & 3];
    uint32_t b = (i & 1) ? (word >> 16) : (word & 0xFFFFu);
    if (kAct == MXQ_ACT_GELU_TANH) b = gelu_bf16(b);
    if (kAct == MXQ_ACT_SWIGLU) {
      const uint32_t uw = up[i >> 3][(i >> 1) & 3];
      b = swiglu_bf16(b, (i & 1) ? (uw >> 16) : (uw & 0xFFFFu));
    }
    v[i] = (double)bf16_to_f32(b);
  }
}

// v of the lane that DPP control kCtrl selects, through moves of the two halves: no LDS
// traffic, unlike a general lane shuffle. quad_perm 0xB1 / 0x4E / 0x1B give lane ^ 1 / ^ 2 / ^ 3
// within each quad, row_ror:8 (0x128) lane ^ 8 within each 16-lane row, row_half_mirror (0x141)
// lane ^ 7 within each 8-lane half.
template <int kCtrl>
MXQ_DEVICE double dpp_f64(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const int lo = __builtin_amdgcn_mov_dpp((int)(uint32_t)b, kCtrl, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_mov_dpp((int)(uint32_t)(b >> 32), kCtrl, 0xF, 0xF, false);
  return __builtin_bit_cast(double, ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

// One radix-4 step across the four lanes i, i ^ m, i ^ 2m, i ^ 3m holding x_k (k the lane's digit):
// y_k = S - 2 x_{k^3} = (x_k + x_{k^1}) + (x_{k^2} - x_{k^3}), i.e. t + (u of lane ^ 2m) with
// t = x + x', u = x - x', x' the value of lane ^ m: two exchanges instead of three.
MXQ_DEVICE double h4_cross(double x, double partner, double u_of_2m) { return (x + partner) + u_of_2m; }

// The unscaled rotation (x @ H_G * sqrt(G)) of the 16 values of each lane, where lane l of the
// wave holds columns 16 l .. 16 l + 15 of a 1024-column window: digits 0 and 1 of the in-group
// index are inside the lane (h4_quad), digit d >= 2 is lane bit pair d - 2 (exchanges with lane
// ^ m and ^ 2m, m = 4^(d-2); DPP moves for d = 2, 3). All lanes of the wave must call it (the
// exchanges are wave-wide).
MXQ_DEVICE void rotate16(double* v, int digits) {
  if (digits >= 1) {
#pragma unroll
    for (int j = 0; j < 16; j += 4) h4_quad(v[j], v[j + 1], v[j + 2], v[j + 3]);
  }
  if (digits >= 2) {
#pragma unroll
    for (int j = 0; j < 4; ++j) h4_quad(v[j], v[j + 4], v[j + 8], v[j + 12]);
  }
  if (digits >= 3) {  // digit 2: lane bits 0-1, within a DPP quad
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const double p = dpp_f64<0xB1>(v[j]);  // lane ^ 1
      v[j] = h4_cross(v[j], p, dpp_f64<0x4E>(v[j] - p));  // u of lane ^ 2
    }
  }
  if (digits >= 4) {  // digit 3: lane bits 2-3; lane ^ 4 = (lane ^ 7) ^ 3, lane ^ 8 a row rotation
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const double p = dpp_f64<0x1B>(dpp_f64<0x141>(v[j]));
      v[j] = h4_cross(v[j], p, dpp_f64<0x128>(v[j] - p));
    }
  }
  for (int d = 4; d < digits; ++d) {
    const int m = 1 << (2 * (d - 2));
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const double p = __shfl_xor(v[j], m, kWave);
      v[j] = h4_cross(v[j], p, __shfl_xor(v[j] - p, 2 * m, kWave));
    }
  }
}

}  // namespace mxq
