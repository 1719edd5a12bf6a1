// Shared device helpers for the gfx950 quantized-linear kernels.
//
// Number formats follow the reference's eager PyTorch semantics
// (backends/turbo/vendor/comfy_kitchen/backends/eager/quantization.py):
// every float operation is one IEEE-754 fp32 operation with round-to-nearest-even,
// bfloat16/float16 results are rounded from fp32 with round-to-nearest-even.
// All HIP sources are compiled with -ffp-contract=off so that no multiply-add
// is fused unless written as fmaf() explicitly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

#include "../../include/mx_qlinear.h"

#define MXQ_DEVICE __device__ __forceinline__

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));

namespace mxq {

constexpr int kWave = 64;

// static_for<N>(f) calls f(std::integral_constant<int, 0>{}) ... f(integral_constant<N-1>): a
// loop whose index is a compile-time constant in every body.
template <typename F, int... Is>
MXQ_DEVICE void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
MXQ_DEVICE void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// ---- bfloat16 / float16 -------------------------------------------------------

MXQ_DEVICE float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// Materialise an fp32 value before it is narrowed. The reference rounds every product to
// fp32 first and then to the output type (two roundings); without this barrier the backend
// folds fptrunc(fmul) into v_fma_mixlo_f16, a single rounding that differs on fp16 ties.
MXQ_DEVICE float fp32_barrier(float f) {
  __asm__ volatile("" : "+v"(f));
  return f;
}

// fp32 -> bf16 bits, round-to-nearest-even (v_cvt_pk_bf16_f32 under the default rounding
// mode). NaN inputs give a quiet NaN; their bit pattern is not part of the contract.
MXQ_DEVICE uint32_t f32_to_bf16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)fp32_barrier(f));
}

// Two fp32 -> packed bf16 pair (lo in bits 0..15), one v_cvt_pk_bf16_f32.
MXQ_DEVICE uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  typedef float f2 __attribute__((ext_vector_type(2)));
  const f2 v = {fp32_barrier(lo), fp32_barrier(hi)};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf2));
}

// f rounded to bfloat16 (round-to-nearest-even), as an fp32 value: one v_cvt_pk_bf16_f32 with the
// value in the high half and zero in the low half, so the word already is the fp32 form (no
// unpacking shift). Rounding each value of a pair this way costs two instructions where a packed
// conversion and the two unpacks cost three.
MXQ_DEVICE float round_bf16(float f) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  typedef float f2 __attribute__((ext_vector_type(2)));
  const f2 v = {0.0f, fp32_barrier(f)};
  return __builtin_bit_cast(float, __builtin_convertvector(v, bf2));
}

// Two bf16-valued fp32 numbers (low 16 bits zero) as one packed pair, lo in bits 0..15.
MXQ_DEVICE uint32_t pair_of_rounded(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

MXQ_DEVICE float f16_to_f32(uint32_t bits16) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
  return (float)h;
}

MXQ_DEVICE uint32_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)fp32_barrier(f);  // v_cvt_f16_f32, round-to-nearest-even
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

MXQ_DEVICE float round_f16(float f) { return f16_to_f32(f32_to_f16_bits(f)); }

// Output element types, by the reference's dtype codes
// (backends/eager/quantization.py:34-42): 0 fp32, 1 fp16, 2 bf16.
template <int kCode> struct OutT;
template <> struct OutT<0> {
  typedef float T;
  static MXQ_DEVICE float round(float f) { return f; }
  static MXQ_DEVICE float load(const float* p) { return *p; }
};
template <> struct OutT<1> {
  typedef uint16_t T;
  static MXQ_DEVICE float round(float f) { return round_f16(f); }
  static MXQ_DEVICE float load(const uint16_t* p) { return f16_to_f32(*p); }
};
template <> struct OutT<2> {
  typedef uint16_t T;
  static MXQ_DEVICE float round(float f) { return round_bf16(f); }
  static MXQ_DEVICE float load(const uint16_t* p) { return bf16_to_f32(*p); }
};

template <int kCode> MXQ_DEVICE void store_out(typename OutT<kCode>::T* p, float v);
template <> MXQ_DEVICE void store_out<0>(float* p, float v) { *p = v; }
template <> MXQ_DEVICE void store_out<1>(uint16_t* p, float v) { *p = (uint16_t)f32_to_f16_bits(v); }
template <> MXQ_DEVICE void store_out<2>(uint16_t* p, float v) { *p = (uint16_t)f32_to_bf16_bits(v); }

// ---- quantizer pieces -----------------------------------------------------------

// Eager scale: max(fp32(amax) / 127, 1e-30) (quantization.py:872-873).
MXQ_DEVICE float row_scale_from_absmax(float amax) {
  float s = amax / 127.0f;
  return (s != s) ? s : fmaxf(s, 1e-30f);
}

// Round a float holding a bf16/fp16/fp32 quotient to int8 with the eager rule:
// round-half-to-even, clamp to [-128, 127]; NaN -> 0.
MXQ_DEVICE int quant_round_clamp(float qf) {
  float r = __builtin_rintf(qf);
  r = fminf(fmaxf(r, -128.0f), 127.0f);
  return (qf != qf) ? 0 : (int)r;
}

// ---- row quantization of packed bf16 values (8 values in 4 words -> 8 int8 in 2 words) ----
MXQ_DEVICE float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
MXQ_DEVICE float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

MXQ_DEVICE uint32_t pack_q4(int a, int b, int c, int d) {
  return (uint32_t)(a & 0xFF) | ((uint32_t)(b & 0xFF) << 8) | ((uint32_t)(c & 0xFF) << 16) |
         ((uint32_t)(d & 0xFF) << 24);
}

// Quantize 8 bf16 values (4 packed words) with reciprocal r; returns 8 int8 in two words.
MXQ_DEVICE v2u quant8_bf16(v4u w, float r) {
  int q[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    q[2 * i] = quant_round_clamp(round_bf16(bf16_lo(w[i]) * r));
    q[2 * i + 1] = quant_round_clamp(round_bf16(bf16_hi(w[i]) * r));
  }
  v2u o;
  o[0] = pack_q4(q[0], q[1], q[2], q[3]);
  o[1] = pack_q4(q[4], q[5], q[6], q[7]);
  return o;
}

// The same for a row whose absmax is finite. Then |bf16(v * r)| <= 127.5 (r = 1 / bf16(s) and
// bf16(s) is within 2^-8 of amax / 127), so the integer n = rne(bf16(v * r)) lies in
// [-128, 128] and only the upper clamp can act. n comes from one fp32 addition of 1.5 * 2^23 (an
// exact sum rounded half to even): the sum's bits are 0x4B400000 + n, so their low 16 bits are n
// as int16. Two such halves share a word, one v_pk_min_i16 clamps both to 127, and the low
// bytes are the two's complement int8 values.
typedef short mxq_s2 __attribute__((ext_vector_type(2)));

// (flo, fhi: the two values already rounded to bf16, as fp32)
MXQ_DEVICE uint32_t quant_pair_finite(float flo, float fhi) {
  constexpr float kRound = 12582912.0f;
  const uint32_t lo = __float_as_uint(flo + kRound), hi = __float_as_uint(fhi + kRound);
  const mxq_s2 n = __builtin_bit_cast(mxq_s2, __builtin_amdgcn_perm(hi, lo, 0x05040100u));
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(n, mxq_s2{127, 127}));
}

MXQ_DEVICE v2u quant8_bf16_finite(v4u w, float r) {
  uint32_t n[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) n[i] = quant_pair_finite(round_bf16(bf16_lo(w[i]) * r), round_bf16(bf16_hi(w[i]) * r));
  v2u o;
  o[0] = __builtin_amdgcn_perm(n[1], n[0], 0x06040200u);
  o[1] = __builtin_amdgcn_perm(n[3], n[2], 0x06040200u);
  return o;
}

MXQ_DEVICE bool finite_absmax(float amax) { return __float_as_uint(amax) < 0x7F800000u; }

// ---- tanh-GELU on bfloat16 ----------------------------------------------------------
// Bit-exact torch CPU gelu(approximate="tanh") on a bfloat16 input (the routine the reference
// applies, backends/turbo/vendor/comfy_kitchen/backends/_activations.py:47-48). The function
// depends on the 16 input bits only: inputs with biased exponent below MXQ_GELU_E_LO map to
// bf16(x / 2), finite inputs at or above MXQ_GELU_E_HI to x (x > 0) or -0.0 (x < 0), +inf to
// +inf and -inf / NaN to MXQ_GELU_NAN; the 3072 inputs in between come from a table generated
// from torch by gen_gelu_table.py, which verifies each rule against all 65,536 torch outputs.
#define MXQ_GELU_TABLE_DECL constexpr uint16_t kGeluTableC[3072]
#include "gelu_tanh_bf16_table.inc"
#undef MXQ_GELU_TABLE_DECL

constexpr uint32_t gelu_rule_c(uint32_t b) {
  const uint32_t e = (b >> 7) & 0xFFu, sign = b & 0x8000u, mag = b & 0x7FFFu;
  if (e < MXQ_GELU_E_LO) {
    // x / 2: one exponent step down, or for e < 2 a right shift of the significand with
    // round-half-to-even.
    const uint32_t v = mag & 0xFFu;
    return sign | (e >= 2 ? mag - 0x80u : (v >> 1) + ((v & 1u) & ((v >> 1) & 1u)));
  }
  if (e < MXQ_GELU_E_HI)
    return kGeluTableC[((b >> 15) * (MXQ_GELU_E_HI - MXQ_GELU_E_LO) + (e - MXQ_GELU_E_LO)) * 128u + (b & 0x7Fu)];
  if (e < 255u) return sign ? 0x8000u : b;
  return b == 0x7F80u ? 0x7F80u : MXQ_GELU_NAN;
}

// The function over all 65,536 inputs (v[b] = gelu(b)), evaluated at compile time: 128 KB in
// global memory that kernels gather from, or that a GEMM epilogue copies into LDS whole.
struct GeluFullTable {
  uint16_t v[65536];
};
constexpr GeluFullTable make_gelu_full() {
  GeluFullTable t{};
  for (uint32_t b = 0; b < 65536u; ++b) t.v[b] = (uint16_t)gelu_rule_c(b);
  return t;
}
static __device__ __attribute__((aligned(16))) const GeluFullTable kGeluFull = make_gelu_full();

MXQ_DEVICE uint32_t gelu_bf16(uint32_t b) { return kGeluFull.v[b & 0xFFFFu]; }

// ---- wave reductions ----------------------------------------------------------------

// Every reduction below needs all 64 lanes active. The exchanges stay inside the VALU (no LDS
// round trip): v_permlane32_swap / v_permlane16_swap of a register with itself leave the two
// halves (rows) in the two results, so their sum is v[i] + v[i ^ 32] (v[i ^ 16]) on every lane;
// the 16-lane steps are DPP operands. row_ror:N makes lane i of a row read lane (i - N) mod 16
// (data rotates towards higher lanes), so row_ror:8 is lane i ^ 8; lane i ^ 4 is lane i + 4 =
// row_ror:12 in banks 0 and 2 (lanes 0-3, 8-11) and lane i - 4 = row_ror:4 in banks 1 and 3;
// quad_perm gives i ^ 2 and i ^ 1.
constexpr int kDppRowRor4 = 0x124, kDppRowRor8 = 0x128, kDppRowRor12 = 0x12C;
constexpr int kDppQuadXor2 = 0x4E, kDppQuadXor1 = 0xB1;  // quad_perm [2,3,0,1], [1,0,3,2]

template <int ctrl>
MXQ_DEVICE uint32_t dpp_lane(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, ctrl, 0xF, 0xF, false);
}
MXQ_DEVICE uint32_t lane_xor4(uint32_t v) {
  const int t = __builtin_amdgcn_update_dpp((int)v, (int)v, kDppRowRor12, 0xF, 0x5, false);
  return (uint32_t)__builtin_amdgcn_update_dpp(t, (int)v, kDppRowRor4, 0xF, 0xA, false);
}

// Sum over the wave with the butterfly pairing i ^ 32, 16, 8, 4, 2, 1 in that order: every lane
// gets the same bits.
MXQ_DEVICE float wave_sum(float v) {
  {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  v += __uint_as_float(dpp_lane<kDppRowRor8>(__float_as_uint(v)));
  v += __uint_as_float(lane_xor4(__float_as_uint(v)));
  v += __uint_as_float(dpp_lane<kDppQuadXor2>(__float_as_uint(v)));
  v += __uint_as_float(dpp_lane<kDppQuadXor1>(__float_as_uint(v)));
  return v;
}

// v + v[i ^ 16] + v[i ^ 32] + v[i ^ 48] on every lane (the four 16-lane rows of the wave).
MXQ_DEVICE float sum_lane_rows(float v) {
  {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Maximum over each 16-lane row.
MXQ_DEVICE uint32_t row16_max_u32(uint32_t v) {
  v = max(v, dpp_lane<kDppRowRor8>(v));
  v = max(v, dpp_lane<kDppRowRor4>(v));
  v = max(v, dpp_lane<kDppQuadXor2>(v));
  return max(v, dpp_lane<kDppQuadXor1>(v));
}

// float64 operands: both words take the same lane.
template <int ctrl>
MXQ_DEVICE double dpp_lane_f64(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint64_t lo = dpp_lane<ctrl>((uint32_t)b), hi = dpp_lane<ctrl>((uint32_t)(b >> 32));
  return __builtin_bit_cast(double, lo | (hi << 32));
}
MXQ_DEVICE double lane_xor4_f64(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint64_t lo = lane_xor4((uint32_t)b), hi = lane_xor4((uint32_t)(b >> 32));
  return __builtin_bit_cast(double, lo | (hi << 32));
}

// Sum over each 16-lane row with the pairing i ^ 1, 2, 4, 8 in that order.
MXQ_DEVICE double row16_sum_f64(double v) {
  v += dpp_lane_f64<kDppQuadXor1>(v);
  v += dpp_lane_f64<kDppQuadXor2>(v);
  v += lane_xor4_f64(v);
  return v + dpp_lane_f64<kDppRowRor8>(v);
}

// Sum over the wave with the pairing i ^ 1, 2, 4, 8, 16, 32 in that order.
MXQ_DEVICE double wave_sum_f64(double v) {
  v = row16_sum_f64(v);
  {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const auto lo = __builtin_amdgcn_permlane16_swap((uint32_t)b, (uint32_t)b, false, false);
    const auto hi = __builtin_amdgcn_permlane16_swap((uint32_t)(b >> 32), (uint32_t)(b >> 32), false, false);
    v = __builtin_bit_cast(double, (uint64_t)lo[0] | ((uint64_t)hi[0] << 32)) +
        __builtin_bit_cast(double, (uint64_t)lo[1] | ((uint64_t)hi[1] << 32));
  }
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const auto lo = __builtin_amdgcn_permlane32_swap((uint32_t)b, (uint32_t)b, false, false);
  const auto hi = __builtin_amdgcn_permlane32_swap((uint32_t)(b >> 32), (uint32_t)(b >> 32), false, false);
  return __builtin_bit_cast(double, (uint64_t)lo[0] | ((uint64_t)hi[0] << 32)) +
         __builtin_bit_cast(double, (uint64_t)lo[1] | ((uint64_t)hi[1] << 32));
}

// Integer sum over the wave (exact in any order).
MXQ_DEVICE int wave_sum_i32(int v) {
  v += (int)dpp_lane<kDppRowRor8>((uint32_t)v);
  v += (int)dpp_lane<kDppRowRor4>((uint32_t)v);
  v += (int)dpp_lane<kDppQuadXor2>((uint32_t)v);
  v += (int)dpp_lane<kDppQuadXor1>((uint32_t)v);
  {
    const auto r = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
    v = (int)(r[0] + r[1]);
  }
  const auto r = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
  return (int)(r[0] + r[1]);
}

// Unsigned maximum over the wave (order does not matter for a maximum).
MXQ_DEVICE uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_lane<kDppRowRor8>(v));
  v = max(v, dpp_lane<kDppRowRor4>(v));
  v = max(v, dpp_lane<kDppQuadXor2>(v));
  v = max(v, dpp_lane<kDppQuadXor1>(v));
  {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = max(r[0], r[1]);
  }
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max(r[0], r[1]);
}

// ---- absolute maxima with torch's NaN propagation ----------------------------------------
// |x| as bits: non-negative floats order like their bit patterns and a NaN (sign cleared) sorts
// above +inf, so an integer maximum of these bits is |x|'s maximum with NaN propagated, as
// torch's amax does (an IEEE fmax would drop the NaN).
MXQ_DEVICE uint32_t abs_bits(float x) { return __float_as_uint(x) & 0x7FFFFFFFu; }

typedef unsigned short mxq_us2 __attribute__((ext_vector_type(2)));

// Running maximum of |bf16| over packed pairs: both halves at once (v_pk_max_u16).
MXQ_DEVICE uint32_t absmax_acc_bf16x2(uint32_t acc, uint32_t w) {
  const mxq_us2 m = __builtin_elementwise_max(__builtin_bit_cast(mxq_us2, acc),
                                              __builtin_bit_cast(mxq_us2, w & 0x7FFF7FFFu));
  return __builtin_bit_cast(uint32_t, m);
}

// The float bits of the larger half of such a packed accumulator.
MXQ_DEVICE uint32_t absmax_bits_of_bf16x2(uint32_t acc) {
  const uint32_t lo = acc & 0xFFFFu, hi = acc >> 16;
  return (lo > hi ? lo : hi) << 16;
}

// Maximum of absolute-value bits across the wave, returned as the float.
MXQ_DEVICE float wave_absmax(uint32_t bits) { return __uint_as_float(wave_max_u32(bits)); }

// Non-negative floats order like their bit patterns; NaN (0x7FC00000) sorts above +inf.
MXQ_DEVICE void atomic_max_nonneg(float* addr, float v) {
  atomicMax(reinterpret_cast<unsigned int*>(addr), __float_as_uint(v));
}

// ---- direct-to-LDS pipelines -------------------------------------------------------

typedef const void __attribute__((address_space(1)))* gptr_t;
typedef void __attribute__((address_space(3)))* lptr_t;

// Direct-to-LDS 16-byte buffer load: lane l's 16 bytes from base + voff + soff land at
// dst + 16 l (dst wave-uniform). The raw buffer (stride 0) spans `bytes` bytes, so the caller's
// per-lane offset is a fixed 32-bit register and the advance along K a scalar offset: unlike a
// global load, no 64-bit address is formed per load. (The buffer intrinsics stay inside device
// functions: a kernel body naming them directly gets no host-side launch stub.)
constexpr int kRawBufferWord3 = 0x00020000;  // resource word 3: 32-bit data format, no swizzle
MXQ_DEVICE void buffer_load_lds16(const void* base, int bytes, lptr_t dst, uint32_t voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, kRawBufferWord3), dst, 16, (int)voff,
      soff, 0, 0);
}

// 16-byte buffer load into registers from a raw buffer of `bytes` bytes at `base` (wave-uniform):
// an offset at or beyond `bytes` reads zeros, so a lane with nothing to read passes such an offset
// instead of branching around the load and zeroing its registers.
MXQ_DEVICE v4u buffer_load_x4(const void* base, int bytes, uint32_t voff) {
  return __builtin_amdgcn_raw_buffer_load_b128(
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, kRawBufferWord3), (int)voff, 0, 0);
}
constexpr uint32_t kBufferOff = 0x80000000u;  // an offset beyond every buffer these kernels form

// s_waitcnt with vmcnt <= n (lgkmcnt and expcnt left alone); n is a compile-time constant.
template <int n> MXQ_DEVICE void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// s_waitcnt vmcnt(n) lgkmcnt(0).
template <int n> MXQ_DEVICE void wait_vm_lgkm0() {
  static_assert(n >= 0 && n < 64, "vmcnt is six bits");
  __builtin_amdgcn_s_waitcnt((n & 0xF) | ((n >> 4) << 14) | (0x7 << 4));
}

// s_waitcnt vmcnt(0) lgkmcnt(0).
MXQ_DEVICE void wait_all() { __builtin_amdgcn_s_waitcnt(0x0070); }

// s_waitcnt lgkmcnt(n): all but the n most recent LDS reads have completed (n <= 15).
template <int n> MXQ_DEVICE void wait_lgkm() { __builtin_amdgcn_s_waitcnt(0xC07F | (n << 8)); }
MXQ_DEVICE void wait_lgkm8() { wait_lgkm<8>(); }

// Workgroup barrier without the implicit drain of __syncthreads(): loads in flight stay in
// flight. The empty asm statements keep the compiler from moving memory accesses across it
// (the barrier intrinsic itself is not a memory operation to the optimiser); the hardware
// ordering comes from the s_waitcnt that precedes each call.
MXQ_DEVICE void barrier_no_drain() {
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}

// ds_read_b128 / ds_read_b64 issued as inline assembly, so that the compiler's wait-count pass
// does not see them: with direct-to-LDS loads in flight that pass only ever waits for LDS reads
// with lgkmcnt(0), which would serialise every fragment read with the MFMAs it should overlap.
// A kernel using them places its LDS waits itself (wait_lgkm / wait_all) and follows each such
// wait with __builtin_amdgcn_sched_barrier(0): the compiler sees no dependence between the wait
// and the registers it covers, so without the barrier it may schedule their first use above it.
// Every destination dword must also be used after that wait: the compiler takes the result as
// written when the asm issues, so a dword with no later use may be handed to another value while
// the read is in flight, and the read's late write then corrupts that value (an address, say).
template <int kOff>
MXQ_DEVICE v4i lds_read_b128(uint32_t addr) {
  v4i r;
  __asm__ volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(kOff));
  return r;
}

// LDS writes issued as inline assembly, for the same reason: code that runs while direct-to-LDS
// loads are in flight (a tile's epilogue behind the next tile's first operand loads) would
// otherwise wait for all of them before its first LDS access. The "memory" clobber keeps them in
// program order with the other memory accesses; one wave's LDS instructions execute in order, so
// a later read by the same wave sees them without a wait.
MXQ_DEVICE void lds_write_b32(uint32_t addr, uint32_t v) {
  __asm__ volatile("ds_write_b32 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
MXQ_DEVICE void lds_write_b64(uint32_t addr, v2u v) {
  __asm__ volatile("ds_write_b64 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
MXQ_DEVICE void lds_write_b128(uint32_t addr, v4u v) {
  __asm__ volatile("ds_write_b128 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
MXQ_DEVICE uint32_t lds_read_b32(uint32_t addr) {
  uint32_t r;
  __asm__ volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(addr) : "memory");
  return r;
}
MXQ_DEVICE uint32_t lds_read_u16_at(uint32_t addr) {  // zero-extended
  uint32_t r;
  __asm__ volatile("ds_read_u16 %0, %1" : "=v"(r) : "v"(addr) : "memory");
  return r;
}
MXQ_DEVICE uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(lptr_t)const_cast<void*>(p); }

}  // namespace mxq

// ---- host-side error plumbing (defined in capi.hip) -------------------------------
int mxq_set_error(int code, const char* fmt, ...);
int mxq_check_launch(const char* what);
int mxq_cu_count();  // compute units of the current device

// Workgroups of one kernel resident per CU, from the occupancy query, cached per (kernel,
// device, block, dynamic LDS): the query costs host time on every launch otherwise.
int mxq_blocks_per_cu(const void* kernel, int block, size_t lds);

// Workgroups of `kernel` that are resident at once on the current device (for grid-stride
// kernels whose workgroups each take an equal share of the rows: a grid larger than this leaves
// its last workgroups to start when the first have finished), capped at `want`.
template <class K>
inline unsigned mxq_resident_grid(K kernel, int block, size_t lds, int64_t want) {
  const int64_t cap = (int64_t)mxq_blocks_per_cu(reinterpret_cast<const void*>(kernel), block, lds) * mxq_cu_count();
  return (unsigned)(want < cap ? want : cap);
}
