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

// The compact form, for kernels with 8 KB of LDS to spare rather than 128 KB: the 3840 entries
// of biased exponents [E_LO, E_NEG), both signs (entry (b >> 15) * span + (b & 0x7FFF) - E_LO * 128),
// padded to 8 KB. silu_compact_offset(b) is the byte offset of b's entry when silu_compact_in(b),
// else some offset inside the table; silu_rule_out(b) is the value of every b outside the range
// (silu_rule_c's other rules). Checked against all 65,536 torch outputs by the GPU tests of the
// SwiGLU epilogue and, on the CPU, by tests/test_oracle_convrot.py.
constexpr uint32_t kSiluLoMag = (uint32_t)MXQ_SILU_E_LO << 7;
constexpr uint32_t kSiluSpan = (uint32_t)(MXQ_SILU_E_NEG - MXQ_SILU_E_LO) << 7;
struct SiluCompactTable {
  uint16_t v[4096];
};
constexpr SiluCompactTable make_silu_compact() {
  SiluCompactTable t{};
  for (uint32_t i = 0; i < 2u * kSiluSpan; ++i) t.v[i] = kSiluTableC[i];
  return t;
}
static_assert(2u * kSiluSpan == MXQ_SILU_TABLE_SIZE && MXQ_SILU_TABLE_SIZE <= 4096, "compact SiLU table layout");
static __device__ __attribute__((aligned(16))) const SiluCompactTable kSiluCompact = make_silu_compact();

MXQ_DEVICE bool silu_compact_in(uint32_t b) { return (b & 0x7FFFu) - kSiluLoMag < kSiluSpan; }
MXQ_DEVICE uint32_t silu_compact_offset(uint32_t b) {
  const uint32_t off = min((b & 0x7FFFu) - kSiluLoMag, kSiluSpan - 1u);  // below the range: wraps, clamped
  return ((b >> 15) * kSiluSpan + off) * 2u;
}
MXQ_DEVICE uint32_t silu_rule_out(uint32_t b) {
  const uint32_t e = (b >> 7) & 0xFFu, sign = b & 0x8000u, mag = b & 0x7FFFu;
  if (e < MXQ_SILU_E_LO) {
    const uint32_t v = mag & 0xFFu;
    return sign | (e >= 2 ? mag - 0x80u : (v >> 1) + ((v & 1u) & ((v >> 1) & 1u)));
  }
  if (e == 255u) return b == 0x7F80u ? 0x7F80u : MXQ_SILU_NAN;
  return sign ? 0x8000u : b;  // e >= E_NEG: x (positive) or -0.0
}

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

// One radix-4 step across the four lanes i, i ^ m, i ^ 2m, i ^ 3m holding x_k (k the lane's digit):
// y_k = S - 2 x_{k^3} = (x_k + x_{k^1}) + (x_{k^2} - x_{k^3}), i.e. t + (u of lane ^ 2m) with
// t = x + x', u = x - x', x' the value of lane ^ m: two exchanges instead of three.
MXQ_DEVICE double h4_cross(double x, double partner, double u_of_2m) { return (x + partner) + u_of_2m; }

// A wave's transpose buffer: per 16-lane group a 16 x 16 matrix of doubles with rows of 18
// (144 bytes: sixteen rows written at one 16-byte slot start on sixteen distinct bank groups), and
// 16 doubles between groups (the two groups of a half-wave read one row each on disjoint banks).
// Every access is a per-lane base plus a constant offset.
constexpr int kTRow = 18;
constexpr int kTGroup = 16 * kTRow + 16;
constexpr int kTWave = 4 * kTGroup;  // doubles per wave

// Lanes of one wave exchange data through its own LDS region: the hardware performs a wave's LDS
// operations in order, so only the compiler must keep each write above the reads of other lanes.
MXQ_DEVICE void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The unscaled rotation (x @ H_G * sqrt(G)) of the 16 values of each lane, where lane l of the
// wave holds columns 16 l .. 16 l + 15 of a 1024-column window: digits 0 and 1 of the in-group
// index are inside the lane, digits 2 and 3 are lane bits 0-1 and 2-3 within a 16-lane group, and
// digit d >= 4 is lane bit pair d - 2. For digits 2 and 3 each 16-lane group transposes its
// 16 x 16 values through the wave's LDS region `tb` (kTWave doubles): lane s then holds value s
// of the group's sixteen lanes, applies both digits in registers with the same radix-4 step as
// digits 0 and 1, and the transpose is undone. Digits >= 4 (G >= 1024) exchange with __shfl_xor.
// All lanes of the wave must call it.
MXQ_DEVICE void rotate16(double* v, int digits, double* tb) {
  if (digits >= 1) {
#pragma unroll
    for (int j = 0; j < 16; j += 4) h4_quad(v[j], v[j + 1], v[j + 2], v[j + 3]);
  }
  if (digits >= 2) {
#pragma unroll
    for (int j = 0; j < 4; ++j) h4_quad(v[j], v[j + 4], v[j + 8], v[j + 12]);
  }
  if (digits >= 3) {
    const int lane = threadIdx.x & 63, s = lane & 15;
    double* gb = tb + (lane >> 4) * kTGroup;
    typedef double d2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int c = 0; c < 8; ++c) *reinterpret_cast<d2*>(gb + s * kTRow + 2 * c) = d2{v[2 * c], v[2 * c + 1]};
    wave_lds_fence();
    double w[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) w[r] = gb[r * kTRow + s];
    wave_lds_fence();
#pragma unroll
    for (int j = 0; j < 16; j += 4) h4_quad(w[j], w[j + 1], w[j + 2], w[j + 3]);  // digit 2
    if (digits >= 4) {
#pragma unroll
      for (int j = 0; j < 4; ++j) h4_quad(w[j], w[j + 4], w[j + 8], w[j + 12]);  // digit 3
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) gb[r * kTRow + s] = w[r];
    wave_lds_fence();
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const d2 pr = *reinterpret_cast<const d2*>(gb + s * kTRow + 2 * c);
      v[2 * c] = pr[0];
      v[2 * c + 1] = pr[1];
    }
    wave_lds_fence();
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
