// Per-token INT8 quantizers and adaLN for gfx950.
//
// Row quantizer semantics (backends/turbo/vendor/comfy_kitchen/backends/eager/quantization.py:857-875):
//   amax = max |x|;  s = max(fp32(amax) / 127, 1e-30);  q = clamp(rne(T(x / T(s))), -128, 127)
// where T is the input dtype (bf16 / fp16 / fp32) and the division is one fp32 division rounded
// to T. For bf16 the quotient of two bf16 values is never within 2^-17 (relative) of a bf16
// rounding midpoint unless it is exactly representable, so bf16(x * rn(1/s)) == bf16(x / s)
// for every pair; the bf16 kernels therefore take one reciprocal per row and multiply.
// (The identity is checked exhaustively over all bf16 pairs by the CPU test suite.)
//
// Layout of the row quantizers: one wavefront per row; each lane owns 16-byte chunks lane,
// lane+64, ... of the row, held in registers between the absmax reduction and the quantize pass,
// so x is read from HBM exactly once and q written once (the memory-bound roofline: 2 B read +
// 1 B written / element). The quantizer fed a known row absmax and the adaLN kernels below
// describe their own layouts.

#include "act_f16.h"

namespace mxq {

constexpr int kQuantBlock = 256;               // 4 waves, one row each
constexpr int kRowsPerBlock = kQuantBlock / kWave;

MXQ_DEVICE uint32_t gelu_pair(uint32_t w) {
  return gelu_bf16(w & 0xFFFFu) | (gelu_bf16(w >> 16) << 16);
}


// bf16 rows, cols % 8 == 0, cols <= 512 * NCH: row held in registers.
template <int NCH, bool kGelu>
__global__ __launch_bounds__(kQuantBlock) void quant_rows_bf16_reg(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q, float* __restrict__ scales,
    int64_t rows, int cols) {
  const int lane = threadIdx.x % kWave;
  const int nchunk = cols / 8;
  for (int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave; row < rows;
       row += (int64_t)gridDim.x * kRowsPerBlock) {
    const v4u* src = reinterpret_cast<const v4u*>(x + row * cols);
    v4u v[NCH];
    uint32_t m = 0;
    // All of the row's loads are issued before any is used (a chunk past the row end re-reads
    // the row's last chunk and is masked below): with a load inside a branch the compiler waited
    // for each load before issuing the next.
#pragma unroll
    for (int j = 0; j < NCH; ++j) v[j] = __builtin_nontemporal_load(src + min(lane + j * kWave, nchunk - 1));
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const bool ok = lane + j * kWave < nchunk;
      if (kGelu) {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[j][i] = gelu_pair(v[j][i]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) m = ok ? absmax_acc_bf16x2(m, v[j][i]) : m;
    }
    const float amax = wave_absmax(absmax_bits_of_bf16x2(m));
    const float s = row_scale_from_absmax(amax);
    const float r = 1.0f / round_bf16(s);
    v2u* dst = reinterpret_cast<v2u*>(q + row * cols);
    if (finite_absmax(amax)) {
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        const int c = lane + j * kWave;
        if (c < nchunk) __builtin_nontemporal_store(quant8_bf16_finite(v[j], r), dst + c);
      }
    } else {
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        const int c = lane + j * kWave;
        if (c < nchunk) __builtin_nontemporal_store(quant8_bf16(v[j], r), dst + c);
      }
    }
    if (lane == 0) scales[row] = s;
  }
}

// Any dtype, any cols: two passes over the row with scalar loads (second pass hits cache).
// kNoise: stochastic rounding (quantization.py:803-826): the scaled value, rounded to the input
// dtype, gets noise[row, i] (a uniform draw in the input dtype) added in that dtype, then floor
// and clamp; NaN -> 0.
template <int kDtype, bool kGelu, bool kNoise = false>
__global__ __launch_bounds__(kQuantBlock) void quant_rows_generic(
    const void* __restrict__ xv, int8_t* __restrict__ q, float* __restrict__ scales,
    int64_t rows, int64_t cols, const void* __restrict__ noise = nullptr) {
  const int lane = threadIdx.x % kWave;
  for (int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave; row < rows;
       row += (int64_t)gridDim.x * kRowsPerBlock) {
    auto load = [&](int64_t i) -> float {
      float f;
      if (kDtype == MXQ_DTYPE_F32) {
        f = reinterpret_cast<const float*>(xv)[row * cols + i];
      } else {
        uint32_t b = reinterpret_cast<const uint16_t*>(xv)[row * cols + i];
        if (kGelu) b = (kDtype == MXQ_DTYPE_BF16) ? gelu_bf16(b) : gelu_f16(b);
        f = (kDtype == MXQ_DTYPE_BF16) ? bf16_to_f32(b) : f16_to_f32(b);
      }
      return f;
    };
    uint32_t m = 0;
    for (int64_t i = lane; i < cols; i += kWave) {
      const uint32_t b = abs_bits(load(i));
      m = m > b ? m : b;
    }
    const float amax = wave_absmax(m);
    const float s = row_scale_from_absmax(amax);
    float s_math;
    if (kDtype == MXQ_DTYPE_BF16) {
      s_math = round_bf16(s);
    } else if (kDtype == MXQ_DTYPE_F16) {
      s_math = round_f16(s);
      if (s_math == 0.0f) s_math = 6.103515625e-05f;  // torch.finfo(float16).tiny
    } else {
      s_math = s;
    }
    for (int64_t i = lane; i < cols; i += kWave) {
      const float f = load(i);
      float qf = f / s_math;
      if (kDtype == MXQ_DTYPE_BF16) qf = round_bf16(qf);
      if (kDtype == MXQ_DTYPE_F16) qf = round_f16(qf);
      if constexpr (kNoise) {
        float r;
        if (kDtype == MXQ_DTYPE_F32) {
          r = reinterpret_cast<const float*>(noise)[row * cols + i];
        } else {
          const uint16_t b = reinterpret_cast<const uint16_t*>(noise)[row * cols + i];
          r = (kDtype == MXQ_DTYPE_BF16) ? bf16_to_f32(b) : f16_to_f32(b);
        }
        float t = qf + r;
        if (kDtype == MXQ_DTYPE_BF16) t = round_bf16(t);
        if (kDtype == MXQ_DTYPE_F16) t = round_f16(t);
        const float fl = fminf(fmaxf(floorf(t), -128.0f), 127.0f);
        q[row * cols + i] = (int8_t)(t != t ? 0 : (int)fl);
      } else {
        q[row * cols + i] = (int8_t)quant_round_clamp(qf);
      }
    }
    if (lane == 0) scales[row] = s;
  }
}

// Streaming quantizer with a known row absmax: a 256-thread workgroup per row (grid-stride only
// beyond 2^31 - 1 rows), the row's scale formed once; thread t takes the row's 16-byte chunks t, t + 256, ...,
// issuing kBatch loads before their stores so that up to kBatch x 4 KB of a row are in flight.
constexpr int kAbsmaxBatch = 10;

// One row's pass: kFinite selects the quantization of a row whose absmax is finite.
template <bool kFinite>
MXQ_DEVICE void absmax_row_pass(const v4u* __restrict__ src, v2u* __restrict__ dst, int chunks, float r, int t) {
  auto quant = [&](v4u w) { return kFinite ? quant8_bf16_finite(w, r) : quant8_bf16(w, r); };
  int c = t;
  for (; c + (kAbsmaxBatch - 1) * 256 < chunks; c += kAbsmaxBatch * 256) {
    v4u w[kAbsmaxBatch];
#pragma unroll
    for (int u = 0; u < kAbsmaxBatch; ++u) w[u] = __builtin_nontemporal_load(src + c + u * 256);
#pragma unroll
    for (int u = 0; u < kAbsmaxBatch; ++u) __builtin_nontemporal_store(quant(w[u]), dst + c + u * 256);
  }
  for (; c < chunks; c += 256) __builtin_nontemporal_store(quant(__builtin_nontemporal_load(src + c)), dst + c);
}

__global__ __launch_bounds__(256) void quant_rows_bf16_absmax(
    const uint16_t* __restrict__ x, const float* __restrict__ row_absmax,
    int8_t* __restrict__ q, float* __restrict__ scales, int64_t rows, int chunks_per_row) {
  const int t = threadIdx.x;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const float amax = row_absmax[row];
    const float s = row_scale_from_absmax(amax);
    const float r = 1.0f / round_bf16(s);
    const v4u* src = reinterpret_cast<const v4u*>(x + row * (int64_t)chunks_per_row * 8);
    v2u* dst = reinterpret_cast<v2u*>(q + row * (int64_t)chunks_per_row * 8);
    if (finite_absmax(amax))
      absmax_row_pass<true>(src, dst, chunks_per_row, r, t);
    else
      absmax_row_pass<false>(src, dst, chunks_per_row, r, t);
    if (t == 0) scales[row] = s;
  }
}

// ---- tanh-GELU + per-token quantizer of wide rows (the FFN intermediate) ----------------
// fc2's quantizer with input_act="gelu_tanh" (CK/backends/_activations.py:40-53 then
// CK/backends/eager/quantization.py:857-875) on fc1's bf16 output y: h = gelu(y), the row's
// absmax of h, q = quantize(h). A persistent grid of one 512-thread workgroup per CU copies the
// 128 KB bf16 -> bf16 GELU table into LDS once (direct-to-LDS loads), then walks rows: thread t
// holds the row's 16-byte chunks t, t + 512, ... in registers (kC of them), with the next row's
// loads in flight behind the current row's work; GELU is one 16-bit LDS read per element; the
// absmax is an integer max over |h| bit patterns (NaN above +inf), reduced over each wave by
// shuffles and over the eight waves through LDS (double-buffered by row parity, so one barrier
// per row); the row is quantized from registers with its scale formed once. With kStoreH, h is
// also written (in place over y is allowed: every element is read before it is written, by the
// same thread, and the prefetched row is a later one).
constexpr int kGeluRowThreads = 512;
constexpr int kGeluRowWaves = kGeluRowThreads / kWave;

template <int kC, bool kStoreH>
__global__ __launch_bounds__(kGeluRowThreads) void quant_rows_gelu_wide(
    const uint16_t* y, int8_t* __restrict__ q, float* __restrict__ scales, uint16_t* h,
    int64_t rows, int chunks) {
  __shared__ __attribute__((aligned(16))) uint16_t tab[65536];
  __shared__ uint32_t red[2][kGeluRowWaves];
  const int t = threadIdx.x, lane = t & (kWave - 1), wave = t >> 6;
  {
    const char* src = reinterpret_cast<const char*>(&kGeluFull) + lane * 16;
    for (int b = wave; b < 128; b += kGeluRowWaves)
      __builtin_amdgcn_global_load_lds((gptr_t)(src + b * 1024), (lptr_t)(reinterpret_cast<char*>(tab) + b * 1024), 16, 0, 0);
  }
  const int64_t stride = gridDim.x;
  // Rows past the end re-read the last row (never used), so every load is issued unconditionally.
  auto load_row = [&](int64_t r, v4u (&v)[kC]) {
    const v4u* src = reinterpret_cast<const v4u*>(y + min(r, rows - 1) * (int64_t)chunks * 8);
#pragma unroll
    for (int j = 0; j < kC; ++j) v[j] = __builtin_nontemporal_load(src + min(t + j * kGeluRowThreads, chunks - 1));
  };
  // A row's int8 results stay in registers until the next row's data has landed: its stores are
  // issued then, a whole row of work before the next wait, rather than right before it (waits on
  // the vector-memory counter cover every older access, stores included).
  v2u qv[kC];
  float qs = 0.0f;
  auto store_q = [&](int64_t r) {
    v2u* dq = reinterpret_cast<v2u*>(q + r * (int64_t)chunks * 8);
#pragma unroll
    for (int j = 0; j < kC; ++j) {
      const int c = t + j * kGeluRowThreads;
      if (c < chunks) __builtin_nontemporal_store(qv[j], dq + c);
    }
    if (t == 0) scales[r] = qs;
  };
  auto do_row = [&](int64_t r, v4u (&v)[kC], int parity) {
    uint32_t m = 0;
#pragma unroll
    for (int j = 0; j < kC; ++j) {
      const bool ok = t + j * kGeluRowThreads < chunks;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t w = v[j][i];
        const uint32_t g = (uint32_t)tab[w & 0xFFFFu] | ((uint32_t)tab[w >> 16] << 16);
        v[j][i] = g;
        m = ok ? absmax_acc_bf16x2(m, g) : m;
      }
    }
    uint32_t bits = wave_max_u32(absmax_bits_of_bf16x2(m));
    if (lane == 0) red[parity][wave] = bits;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kGeluRowWaves; ++w) bits = max(bits, red[parity][w]);
    const float amax = __uint_as_float(bits);
    const float s = row_scale_from_absmax(amax);
    const float rcp = 1.0f / round_bf16(s);
    v4u* dh = reinterpret_cast<v4u*>(h + r * (int64_t)chunks * 8);
    if (finite_absmax(amax)) {
#pragma unroll
      for (int j = 0; j < kC; ++j) qv[j] = quant8_bf16_finite(v[j], rcp);
    } else {
#pragma unroll
      for (int j = 0; j < kC; ++j) qv[j] = quant8_bf16(v[j], rcp);
    }
    qs = s;
    if (kStoreH) {
#pragma unroll
      for (int j = 0; j < kC; ++j) {
        const int c = t + j * kGeluRowThreads;
        if (c < chunks) __builtin_nontemporal_store(v[j], dh + c);
      }
    }
  };
  v4u a[kC], b[kC];
  int64_t row = blockIdx.x;
  load_row(row, a);
  int parity = 0;
  int64_t prev = -1;  // the row whose int8 results wait in qv
  // One step: the current row has landed (and every older access has completed: the previous
  // row's prefetch a row of work ago, the stores before it), the held results are stored, the
  // next row's loads go out, and the current row is processed.
  auto step = [&](v4u (&cur)[kC], v4u (&nxt)[kC]) {
    wait_vmcnt<0>();
    if (prev < 0) __syncthreads();  // the table has landed in every wave
    if (prev >= 0) store_q(prev);
    load_row(row + stride, nxt);
    do_row(row, cur, parity);
    prev = row;
    row += stride;
    parity ^= 1;
  };
  while (row < rows) {
    step(a, b);
    if (row >= rows) break;
    step(b, a);
  }
  if (prev >= 0) store_q(prev);
}

// ---- adaLN ------------------------------------------------------------------------
// y = bf16(bf16(bf16(n) * bf16(1 + scale)) + shift), n = (x - mean) * rstd in fp32,
// rstd = 1 / sqrt(var + eps), var the biased variance (CK/backends/eager/adaln.py:11-14 on
// torch's CPU layer_norm). Statistics are two-pass over the register-resident row: the sum on
// the matrix cores (adaln_row_sum), the squared deviations as fp32 fmas. Every adaLN kernel
// forms them with the same operations on the same lane layout (chunk c of 8 values in lane
// c % 64, register c / 64), so a row's result does not depend on which kernel ran it.

// Sum of a row held as chunks v[j] = row chunk lane + 64 j (chunks at or past nchunk are
// zeroed here). Each chunk is a lane's A operand of a 16x16x32 bf16 product with a ones matrix,
// so every output column accumulates the sum of all the wave's values (a zero chunk leaves the
// fp32 accumulator unchanged, so the result does not depend on NCH); lanes l, l ^ 16, l ^ 32 and
// l ^ 48 hold one column's 16 rows. The matrix cores are otherwise idle in these kernels, and
// the VALU, which bounds them, is spared the unpack and two additions per pair.
template <int NCH, bool kAll>
MXQ_DEVICE float adaln_row_sum(v4u (&v)[NCH], int lane, int nchunk) {
  const v8bf ones = __builtin_bit_cast(v8bf, v4u{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
  v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    if (!kAll && lane + j * kWave >= nchunk) v[j] = v4u{0u, 0u, 0u, 0u};
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, v[j]), ones, acc, 0, 0, 0);
  }
  return sum_lane_rows((acc[0] + acc[1]) + (acc[2] + acc[3]));
}

MXQ_DEVICE uint32_t modulate(float xv, float mean, float rstd, uint32_t sc, uint32_t sh) {
  const float n = round_bf16((xv - mean) * rstd);
  const float t = round_bf16(1.0f + bf16_to_f32(sc));
  const float p = round_bf16(n * t);
  return f32_to_bf16_bits(p + bf16_to_f32(sh));
}

// The same with t = bf16(1 + scale) given.
MXQ_DEVICE uint32_t modulate_t(float xv, float mean, float rstd, float t, uint32_t sh) {
  const float n = round_bf16((xv - mean) * rstd);
  const float p = round_bf16(n * t);
  return f32_to_bf16_bits(p + bf16_to_f32(sh));
}

// One row of adaLN (+ quant) with the row in registers. kLds: the modulation comes from LDS,
// t = bf16(1 + scale) already formed; otherwise from global memory, t formed here.
template <int NCH, bool kQuant, bool kLds>
MXQ_DEVICE void adaln_row(const uint16_t* __restrict__ x, const v4u* scv, const v4u* shv, float eps,
                          int8_t* __restrict__ q, float* __restrict__ scales, uint16_t* __restrict__ y_out,
                          int64_t row, int cols, int lane) {
  const int nchunk = cols / 8;
  const v4u* src = reinterpret_cast<const v4u*>(x + row * cols);
  v4u v[NCH];
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = lane + j * kWave;
    if (c < nchunk) v[j] = __builtin_nontemporal_load(src + c);
  }
  const float mean = adaln_row_sum<NCH, false>(v, lane, nchunk) / (float)cols;
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = lane + j * kWave;
    if (c < nchunk) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = bf16_lo(v[j][i]) - mean, b = bf16_hi(v[j][i]) - mean;
        ss = __builtin_fmaf(a, a, ss);
        ss = __builtin_fmaf(b, b, ss);
      }
    }
  }
  const float var = wave_sum(ss) / (float)cols;
  const float rstd = 1.0f / sqrtf(var + eps);
  uint32_t m = 0;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = lane + j * kWave;
    if (c < nchunk) {
      const v4u sc = scv[c], sh = shv[c];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t lo, hi;
        if constexpr (kLds) {
          lo = modulate_t(bf16_lo(v[j][i]), mean, rstd, bf16_lo(sc[i]), sh[i] & 0xFFFF);
          hi = modulate_t(bf16_hi(v[j][i]), mean, rstd, bf16_hi(sc[i]), sh[i] >> 16);
        } else {
          lo = modulate(bf16_lo(v[j][i]), mean, rstd, sc[i] & 0xFFFF, sh[i] & 0xFFFF);
          hi = modulate(bf16_hi(v[j][i]), mean, rstd, sc[i] >> 16, sh[i] >> 16);
        }
        v[j][i] = lo | (hi << 16);
        m = absmax_acc_bf16x2(m, v[j][i]);
      }
      if (y_out != nullptr) reinterpret_cast<v4u*>(y_out + row * cols)[c] = v[j];
    }
  }
  if (kQuant) {
    const float amax = wave_absmax(absmax_bits_of_bf16x2(m));
    const float s = row_scale_from_absmax(amax);
    const float r = 1.0f / round_bf16(s);
    v2u* dst = reinterpret_cast<v2u*>(q + row * cols);
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = lane + j * kWave;
      if (c < nchunk) __builtin_nontemporal_store(quant8_bf16(v[j], r), dst + c);
    }
    if (lane == 0) scales[row] = s;
  }
}

// A workgroup takes kAdalnRows consecutive rows, kAdalnRows / 4 per wave. When they all share one
// scale row and one shift row (the common case: one modulation per sample), the workgroup forms
// t = bf16(1 + scale) once and keeps t and shift in LDS; otherwise each row reads its modulation
// from global memory.
constexpr int kAdalnRows = 16;
constexpr int kAdalnMaxCols = 8192;

template <int NCH, bool kQuant>
__global__ __launch_bounds__(kQuantBlock) void adaln_rows_reg(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ scale,
    const uint16_t* __restrict__ shift, int64_t scale_group, int64_t shift_group, float eps,
    int8_t* __restrict__ q, float* __restrict__ scales, uint16_t* __restrict__ y_out,
    int64_t rows, int cols) {
  __shared__ __attribute__((aligned(16))) uint16_t s_t[kAdalnMaxCols];
  __shared__ __attribute__((aligned(16))) uint16_t s_sh[kAdalnMaxCols];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int nchunk = cols / 8;
  for (int64_t r0 = (int64_t)blockIdx.x * kAdalnRows; r0 < rows; r0 += (int64_t)gridDim.x * kAdalnRows) {
    const int64_t r1 = min(r0 + kAdalnRows, rows) - 1;
    const int64_t gs = r0 / scale_group, gh = r0 / shift_group;
    if (gs == r1 / scale_group && gh == r1 / shift_group) {  // uniform over the workgroup
      const v4u* scv = reinterpret_cast<const v4u*>(scale + gs * cols);
      const v4u* shv = reinterpret_cast<const v4u*>(shift + gh * cols);
      __syncthreads();  // the previous run's rows are done with the LDS copy
      for (int c = threadIdx.x; c < nchunk; c += kQuantBlock) {
        const v4u sc = scv[c];
        v4u t;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          t[i] = f32_to_bf16_bits(1.0f + bf16_lo(sc[i])) | (f32_to_bf16_bits(1.0f + bf16_hi(sc[i])) << 16);
        reinterpret_cast<v4u*>(s_t)[c] = t;
        reinterpret_cast<v4u*>(s_sh)[c] = shv[c];
      }
      __syncthreads();
      for (int64_t row = r0 + wave; row <= r1; row += kQuantBlock / kWave)
        adaln_row<NCH, kQuant, true>(x, reinterpret_cast<const v4u*>(s_t), reinterpret_cast<const v4u*>(s_sh), eps,
                                     q, scales, y_out, row, cols, lane);
    } else {
      for (int64_t row = r0 + wave; row <= r1; row += kQuantBlock / kWave)
        adaln_row<NCH, kQuant, false>(x, reinterpret_cast<const v4u*>(scale + (row / scale_group) * cols),
                                      reinterpret_cast<const v4u*>(shift + (row / shift_group) * cols), eps, q,
                                      scales, y_out, row, cols, lane);
    }
  }
}

// adaLN with one modulation row for every row (the common case: one sample per launch). One wave
// per row, rows taken grid-stride by the launch's waves; each wave loads its next row into a
// second register buffer before it processes the current one, so a row's HBM latency overlaps
// the previous row's arithmetic. t = bf16(1 + scale) and shift are staged once per workgroup in
// LDS as fp32 (cols * 8 bytes of dynamic LDS). The statistics and the modulation are the same
// operations, in the same order, as adaln_row's (the chunks past the row end are zeroed before
// the sum); rows whose absmax is finite are quantized by the finite-row path.
// Both bf16 halves of w as fp32, as an inline-asm pair: the compiler cannot reuse an earlier
// unpack of the same word, which would keep a row's unpacked values live (twice the registers of
// the packed row) from one pass to the next.
MXQ_DEVICE void unpack_fresh(uint32_t w, float& lo, float& hi) {
  __asm__ volatile("v_lshlrev_b32 %0, 16, %2\n\tv_and_b32 %1, 0xffff0000, %2" : "=&v"(lo), "=v"(hi) : "v"(w));
}

template <int NCH, bool kQuant, bool kExact>
__global__ __launch_bounds__(kQuantBlock) __attribute__((amdgpu_waves_per_eu(kExact && NCH <= 10 ? 3 : 2))) void adaln_uniform_rows(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ scale, const uint16_t* __restrict__ shift,
    float eps, int8_t* __restrict__ q, float* __restrict__ scales, uint16_t* __restrict__ y_out, int64_t rows,
    int cols) {
  extern __shared__ __attribute__((aligned(16))) float s_mod[];
  float* s_t = s_mod;
  float* s_sh = s_mod + cols;
  for (int c = threadIdx.x; c < cols; c += kQuantBlock) {
    s_t[c] = round_bf16(1.0f + bf16_to_f32(scale[c]));
    s_sh[c] = bf16_to_f32(shift[c]);
  }
  __syncthreads();
  const int lane = threadIdx.x % kWave;
  const int nchunk = kExact ? NCH * kWave : cols / 8;  // kExact: cols == NCH * 512
  const int64_t stride = (int64_t)gridDim.x * (kQuantBlock / kWave);
  int64_t row = (int64_t)blockIdx.x * (kQuantBlock / kWave) + threadIdx.x / kWave;

  // Loads are unconditional (a chunk past the row end re-reads the row's last chunk and is masked
  // out of the statistics, the absmax and the stores): a load inside a branch made the compiler
  // wait for every earlier load before issuing it.
  auto load = [&](v4u (&v)[NCH], int64_t r) {
    const v4u* src = reinterpret_cast<const v4u*>(x + r * cols);
#pragma unroll
    for (int j = 0; j < NCH; ++j) v[j] = __builtin_nontemporal_load(src + min(lane + j * kWave, nchunk - 1));
  };
  auto process = [&](v4u (&v)[NCH], int64_t r) {
    const float mean = adaln_row_sum<NCH, kExact>(v, lane, nchunk) / (float)cols;
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const bool ok = kExact || lane + j * kWave < nchunk;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float xl, xh;
        unpack_fresh(v[j][i], xl, xh);
        const float a = ok ? xl - mean : 0.0f, b = ok ? xh - mean : 0.0f;
        ss = __builtin_fmaf(a, a, ss);
        ss = __builtin_fmaf(b, b, ss);
      }
    }
    const float var = wave_sum(ss) / (float)cols;
    const float rstd = 1.0f / sqrtf(var + eps);
    uint32_t m = 0;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = min(lane + j * kWave, nchunk - 1);
      const bool ok = kExact || lane + j * kWave < nchunk;
      {
        const v4f t0 = reinterpret_cast<const v4f*>(s_t)[2 * c], t1 = reinterpret_cast<const v4f*>(s_t)[2 * c + 1];
        const v4f h0 = reinterpret_cast<const v4f*>(s_sh)[2 * c], h1 = reinterpret_cast<const v4f*>(s_sh)[2 * c + 1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float tl = i < 2 ? t0[2 * i] : t1[2 * i - 4], th = i < 2 ? t0[2 * i + 1] : t1[2 * i - 3];
          const float hl = i < 2 ? h0[2 * i] : h1[2 * i - 4], hh = i < 2 ? h0[2 * i + 1] : h1[2 * i - 3];
          float xl, xh;
          unpack_fresh(v[j][i], xl, xh);
          const float nl = round_bf16((xl - mean) * rstd), nh = round_bf16((xh - mean) * rstd);
          v[j][i] = pack_bf16x2(round_bf16(nl * tl) + hl, round_bf16(nh * th) + hh);
          m = ok ? absmax_acc_bf16x2(m, v[j][i]) : m;
        }
        if (y_out != nullptr && ok) __builtin_nontemporal_store(v[j], reinterpret_cast<v4u*>(y_out + r * cols) + c);
      }
      // one chunk's modulation at a time: the LDS reads of later chunks are not hoisted, which
      // would hold every chunk's t and shift in registers at once
      __builtin_amdgcn_sched_barrier(0);
    }
    if (kQuant) {
      const float amax = wave_absmax(absmax_bits_of_bf16x2(m));
      const float s = row_scale_from_absmax(amax);
      const float rcp = 1.0f / round_bf16(s);
      v2u* dst = reinterpret_cast<v2u*>(q + r * cols);
      if (finite_absmax(amax)) {
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
          const int c = lane + j * kWave;
          if (c < nchunk) __builtin_nontemporal_store(quant8_bf16_finite(v[j], rcp), dst + c);
        }
      } else {
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
          const int c = lane + j * kWave;
          if (c < nchunk) __builtin_nontemporal_store(quant8_bf16(v[j], rcp), dst + c);
        }
      }
      if (lane == 0) scales[r] = s;
    }
  };

  // The next row's loads are unconditional (past the last row they re-read row rows - 1), so the
  // compiler's wait for the current row counts exactly the next row's loads as still in flight.
  v4u a[NCH], b[NCH];
  if (row < rows) load(a, row);
  while (row < rows) {
    const int64_t r1 = row + stride;
    load(b, min(r1, rows - 1));
    process(a, row);
    row = r1;
    if (row >= rows) break;
    const int64_t r2 = row + stride;
    load(a, min(r2, rows - 1));
    process(b, row);
    row = r2;
  }
}

// Elementwise tanh-GELU on bf16 (8 elements per thread when 16-byte aligned).
__global__ __launch_bounds__(256) void gelu_bf16_kernel(const uint16_t* __restrict__ x,
                                                        uint16_t* __restrict__ y, int64_t n,
                                                        int vec) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  if (vec) {
    const int64_t nv = n / 8;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nv; i += stride) {
      v4u w = reinterpret_cast<const v4u*>(x)[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = gelu_pair(w[j]);
      reinterpret_cast<v4u*>(y)[i] = w;
    }
    for (int64_t i = nv * 8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
      y[i] = (uint16_t)gelu_bf16(x[i]);
  } else {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
      y[i] = (uint16_t)gelu_bf16(x[i]);
  }
}

// The input activation on float16 rows: y[r, c] = gelu(x[r, c]) (x [rows, cols]) or
// swiglu(x[r, c], x[r, cols + c]) (x [rows, 2 cols], the [gate | up] halves).
template <int kAct>
__global__ __launch_bounds__(256) void act_f16_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
                                                     int64_t rows, int64_t cols) {
  const int64_t n = rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    if constexpr (kAct == MXQ_ACT_GELU_TANH) {
      y[i] = (uint16_t)gelu_f16(x[i]);
    } else {
      const int64_t r = i / cols, c = i - r * cols;
      y[i] = (uint16_t)swiglu_f16(x[r * 2 * cols + c], x[r * 2 * cols + cols + c]);
    }
  }
}

// adaLN on float16 rows (the reference's layer_norm(x) * (1 + scale) + shift evaluated in
// float16, CK/backends/eager/adaln.py:11-14): n = f16((x - mean) * rstd) with the statistics in
// fp32 (mean = sum / cols, var = sum (x - mean)^2 / cols, rstd = 1 / sqrt(var + eps)),
// y = f16(f16(n * f16(1 + scale)) + shift); optionally the row quantizer of y with the float16
// rule (as quant_rows_generic). One wave per row, rows grid-stride; the row is read from global
// memory once per pass (the later passes hit the caches). Each lane sums its columns in order and
// the wave combines the lanes as wave_sum does.
MXQ_DEVICE uint32_t adaln_f16_value(float xv, float mean, float rstd, uint32_t sc, uint32_t sh) {
  const float n = round_f16((xv - mean) * rstd);
  const float t = round_f16(1.0f + f16_to_f32(sc));
  const float p = round_f16(n * t);
  return f32_to_f16_bits(p + f16_to_f32(sh));
}

__global__ __launch_bounds__(kQuantBlock) void adaln_f16_rows(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ scale, const uint16_t* __restrict__ shift,
    int64_t scale_group, int64_t shift_group, float eps, int8_t* __restrict__ q, float* __restrict__ scales,
    uint16_t* __restrict__ y_out, int64_t rows, int64_t cols) {
  const int lane = threadIdx.x % kWave;
  for (int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave; row < rows;
       row += (int64_t)gridDim.x * kRowsPerBlock) {
    const uint16_t* xr = x + row * cols;
    const uint16_t* sc = scale + (row / scale_group) * cols;
    const uint16_t* sh = shift + (row / shift_group) * cols;
    float sum = 0.0f;
    for (int64_t i = lane; i < cols; i += kWave) sum += f16_to_f32(xr[i]);
    const float mean = wave_sum(sum) / (float)cols;
    float ss = 0.0f;
    for (int64_t i = lane; i < cols; i += kWave) {
      const float d = f16_to_f32(xr[i]) - mean;
      ss = __builtin_fmaf(d, d, ss);
    }
    const float rstd = 1.0f / sqrtf(wave_sum(ss) / (float)cols + eps);
    uint32_t m = 0;
    for (int64_t i = lane; i < cols; i += kWave) {
      const uint32_t y = adaln_f16_value(f16_to_f32(xr[i]), mean, rstd, sc[i], sh[i]);
      if (y_out) y_out[row * cols + i] = (uint16_t)y;
      m = max(m, abs_bits(f16_to_f32(y)));
    }
    if (q) {
      const float s = row_scale_from_absmax(wave_absmax(m));
      float s16 = round_f16(s);
      if (s16 == 0.0f) s16 = 6.103515625e-05f;  // torch.finfo(float16).tiny
      for (int64_t i = lane; i < cols; i += kWave) {
        const uint32_t y = adaln_f16_value(f16_to_f32(xr[i]), mean, rstd, sc[i], sh[i]);
        q[row * cols + i] = (int8_t)quant_round_clamp(round_f16(f16_to_f32(y) / s16));
      }
      if (lane == 0) scales[row] = s;
    }
  }
}

__global__ void fill_f32_kernel(float* __restrict__ p, float value, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = value;
}

static unsigned row_grid(int64_t rows) {
  const int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  return (unsigned)(blocks < 65536 * 4 ? blocks : 65536 * 4);
}

// Smallest register-chunk count covering cols (chunks of 8 elements per lane, 64 lanes).
static int pick_nch(int64_t cols) {
  const int64_t need = (cols / 8 + kWave - 1) / kWave;
  const int options[] = {1, 2, 4, 8, 12, 16, 24, 32, 40};
  for (int o : options)
    if (need <= o) return o;
  return 0;
}

}  // namespace mxq

using namespace mxq;

#define MXQ_NCH_SWITCH(nch, BODY) \
  switch (nch) {                  \
    case 1: { constexpr int N_ = 1; BODY; } break;   \
    case 2: { constexpr int N_ = 2; BODY; } break;   \
    case 4: { constexpr int N_ = 4; BODY; } break;   \
    case 8: { constexpr int N_ = 8; BODY; } break;   \
    case 12: { constexpr int N_ = 12; BODY; } break; \
    case 16: { constexpr int N_ = 16; BODY; } break; \
    case 24: { constexpr int N_ = 24; BODY; } break; \
    case 32: { constexpr int N_ = 32; BODY; } break; \
    case 40: { constexpr int N_ = 40; BODY; } break; \
    default: break;                                  \
  }

#define MXQ_NCH_SWITCH_16(nch, BODY) \
  switch (nch) {                     \
    case 1: { constexpr int N_ = 1; BODY; } break;   \
    case 2: { constexpr int N_ = 2; BODY; } break;   \
    case 4: { constexpr int N_ = 4; BODY; } break;   \
    case 8: { constexpr int N_ = 8; BODY; } break;   \
    case 12: { constexpr int N_ = 12; BODY; } break; \
    case 16: { constexpr int N_ = 16; BODY; } break; \
    default: break;                                  \
  }

// Chunks per thread of the wide GELU quantizer; 0 beyond its register budget.
static int pick_gelu_chunks(int64_t cols) {
  const int64_t need = (cols / 8 + kGeluRowThreads - 1) / kGeluRowThreads;
  return need <= 8 ? (int)need : 0;
}

#define MXQ_GELU_CHUNK_SWITCH(c, BODY)                                          \
  switch (c) {                                                                  \
    case 1: { constexpr int C_ = 1; BODY; } break;                              \
    case 2: { constexpr int C_ = 2; BODY; } break;                              \
    case 3: { constexpr int C_ = 3; BODY; } break;                              \
    case 4: { constexpr int C_ = 4; BODY; } break;                              \
    case 5: { constexpr int C_ = 5; BODY; } break;                              \
    case 6: { constexpr int C_ = 6; BODY; } break;                              \
    case 7: { constexpr int C_ = 7; BODY; } break;                              \
    case 8: { constexpr int C_ = 8; BODY; } break;                              \
    default: break;                                                             \
  }

static int gelu_wide_launch(const void* y, void* h, int8_t* q, float* scales, int64_t rows, int64_t cols,
                            hipStream_t st) {
  const int c = pick_gelu_chunks(cols);
  const int64_t grid = rows < 256 ? rows : 256;  // one workgroup per CU (the table fills 128 KB of LDS)
  if (h) {
    MXQ_GELU_CHUNK_SWITCH(c, (quant_rows_gelu_wide<C_, true><<<(unsigned)grid, kGeluRowThreads, 0, st>>>(
                                  (const uint16_t*)y, q, scales, (uint16_t*)h, rows, (int)(cols / 8))));
  } else {
    MXQ_GELU_CHUNK_SWITCH(c, (quant_rows_gelu_wide<C_, false><<<(unsigned)grid, kGeluRowThreads, 0, st>>>(
                                  (const uint16_t*)y, q, scales, nullptr, rows, (int)(cols / 8))));
  }
  return mxq_check_launch("quant_rows_gelu_wide");
}

extern "C" int mxq_quantize_int8_rowwise_gelu(const void* y_bf16, void* h_bf16, int8_t* q, float* scales,
                                              int64_t rows, int64_t cols, void* stream) {
  if (rows < 0 || cols <= 0) return mxq_set_error(MXQ_ERR_INVALID, "bad shape [%lld, %lld]", (long long)rows, (long long)cols);
  if (rows == 0) return MXQ_OK;
  if (!y_bf16 || !q || !scales) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  if (cols % 8 != 0 || (uintptr_t)y_bf16 % 16 != 0 || (uintptr_t)q % 8 != 0 || (uintptr_t)h_bf16 % 16 != 0)
    return mxq_set_error(MXQ_ERR_UNSUPPORTED, "GELU quantizer needs cols %% 8 == 0 and 16-byte aligned rows");
  if (pick_gelu_chunks(cols) == 0)
    return mxq_set_error(MXQ_ERR_UNSUPPORTED, "GELU quantizer row of %lld columns exceeds %d", (long long)cols,
                         8 * 8 * kGeluRowThreads);
  return gelu_wide_launch(y_bf16, h_bf16, q, scales, rows, cols, (hipStream_t)stream);
}

extern "C" int mxq_quantize_int8_rowwise(const void* x, int x_dtype, int8_t* q, float* scales,
                                         int64_t rows, int64_t cols, int input_act,
                                         void* stream) {
  if (rows < 0 || cols < 0) return mxq_set_error(MXQ_ERR_INVALID, "negative shape");
  if (rows == 0) return MXQ_OK;
  if (cols == 0) return mxq_set_error(MXQ_ERR_INVALID, "quantize_int8_rowwise needs cols > 0");
  if (!x || !q || !scales) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  if (x_dtype != MXQ_DTYPE_BF16 && x_dtype != MXQ_DTYPE_F16 && x_dtype != MXQ_DTYPE_F32)
    return mxq_set_error(MXQ_ERR_UNSUPPORTED, "input dtype code %d", x_dtype);
  if (input_act != MXQ_ACT_NONE && input_act != MXQ_ACT_GELU_TANH)
    return mxq_set_error(MXQ_ERR_INVALID, "unsupported input_act code %d", input_act);
  if (input_act == MXQ_ACT_GELU_TANH && x_dtype == MXQ_DTYPE_F32)
    return mxq_set_error(MXQ_ERR_UNSUPPORTED, "gelu_tanh input_act needs bf16 or fp16 input");
  hipStream_t st = (hipStream_t)stream;
  const bool gelu = input_act == MXQ_ACT_GELU_TANH;
  const bool aligned = ((uintptr_t)x % 16 == 0) && ((uintptr_t)q % 8 == 0);
  const int nch = pick_nch(cols);
  // Large GELU inputs take the wide kernel (the GELU table in LDS, loaded once per CU); the
  // register kernels below gather GELU values from the table in global memory.
  if (gelu && x_dtype == MXQ_DTYPE_BF16 && cols % 8 == 0 && aligned && pick_gelu_chunks(cols) > 0 &&
      rows * cols >= ((int64_t)1 << 24))
    return gelu_wide_launch(x, nullptr, q, scales, rows, cols, st);
  if (x_dtype == MXQ_DTYPE_BF16 && cols % 8 == 0 && aligned && nch > 0 && cols <= INT32_MAX) {
    if (gelu) {
      MXQ_NCH_SWITCH(nch, (quant_rows_bf16_reg<N_, true><<<row_grid(rows), kQuantBlock, 0, st>>>(
                               (const uint16_t*)x, q, scales, rows, (int)cols)));
    } else {
      MXQ_NCH_SWITCH(nch, (quant_rows_bf16_reg<N_, false><<<row_grid(rows), kQuantBlock, 0, st>>>(
                               (const uint16_t*)x, q, scales, rows, (int)cols)));
    }
    return mxq_check_launch("quant_rows_bf16_reg");
  }
  if (x_dtype == MXQ_DTYPE_BF16) {
    if (gelu)
      quant_rows_generic<MXQ_DTYPE_BF16, true><<<row_grid(rows), kQuantBlock, 0, st>>>(x, q, scales, rows, cols);
    else
      quant_rows_generic<MXQ_DTYPE_BF16, false><<<row_grid(rows), kQuantBlock, 0, st>>>(x, q, scales, rows, cols);
  } else if (x_dtype == MXQ_DTYPE_F16) {
    if (gelu)
      quant_rows_generic<MXQ_DTYPE_F16, true><<<row_grid(rows), kQuantBlock, 0, st>>>(x, q, scales, rows, cols);
    else
      quant_rows_generic<MXQ_DTYPE_F16, false><<<row_grid(rows), kQuantBlock, 0, st>>>(x, q, scales, rows, cols);
  } else {
    quant_rows_generic<MXQ_DTYPE_F32, false><<<row_grid(rows), kQuantBlock, 0, st>>>(x, q, scales, rows, cols);
  }
  return mxq_check_launch("quant_rows_generic");
}

extern "C" int mxq_quantize_int8_rowwise_stochastic(const void* x, int x_dtype, const void* noise, int8_t* q,
                                                    float* scales, int64_t rows, int64_t cols, void* stream) {
  if (rows < 0 || cols <= 0) return mxq_set_error(MXQ_ERR_INVALID, "bad shape [%lld, %lld]", (long long)rows, (long long)cols);
  if (rows == 0) return MXQ_OK;
  if (!x || !noise || !q || !scales) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  if (x_dtype != MXQ_DTYPE_BF16 && x_dtype != MXQ_DTYPE_F16 && x_dtype != MXQ_DTYPE_F32)
    return mxq_set_error(MXQ_ERR_INVALID, "unsupported input dtype code %d", x_dtype);
  hipStream_t st = (hipStream_t)stream;
  if (x_dtype == MXQ_DTYPE_BF16)
    quant_rows_generic<MXQ_DTYPE_BF16, false, true><<<row_grid(rows), kQuantBlock, 0, st>>>(x, q, scales, rows, cols, noise);
  else if (x_dtype == MXQ_DTYPE_F16)
    quant_rows_generic<MXQ_DTYPE_F16, false, true><<<row_grid(rows), kQuantBlock, 0, st>>>(x, q, scales, rows, cols, noise);
  else
    quant_rows_generic<MXQ_DTYPE_F32, false, true><<<row_grid(rows), kQuantBlock, 0, st>>>(x, q, scales, rows, cols, noise);
  return mxq_check_launch("quant_rows_generic");
}

extern "C" int mxq_quantize_int8_rowwise_absmax(const void* x_bf16, const float* row_absmax,
                                                int8_t* q, float* scales, int64_t rows,
                                                int64_t cols, void* stream) {
  if (rows < 0 || cols <= 0) return mxq_set_error(MXQ_ERR_INVALID, "bad shape [%lld, %lld]", (long long)rows, (long long)cols);
  if (rows == 0) return MXQ_OK;
  if (!x_bf16 || !row_absmax || !q || !scales) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  if (cols % 8 != 0 || (uintptr_t)x_bf16 % 16 != 0 || (uintptr_t)q % 8 != 0)
    return mxq_set_error(MXQ_ERR_UNSUPPORTED, "absmax quantizer needs cols %% 8 == 0 and aligned rows");
  if (cols / 8 > INT32_MAX) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "row too long");
  // One workgroup per row (measured 10 % faster than a grid-stride over 16 workgroups per CU).
  const int64_t blocks = rows < INT32_MAX ? rows : INT32_MAX;
  quant_rows_bf16_absmax<<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>(
      (const uint16_t*)x_bf16, row_absmax, q, scales, rows, (int)(cols / 8));
  return mxq_check_launch("quant_rows_bf16_absmax");
}

static unsigned adaln_grid(int64_t rows) {
  const int64_t blocks = (rows + kAdalnRows - 1) / kAdalnRows;
  return (unsigned)(blocks < 65536 * 4 ? blocks : 65536 * 4);
}

static int adaln_launch(const void* x, const void* scale, const void* shift, int64_t scale_group,
                        int64_t shift_group, float eps, int8_t* q, float* scales, void* y_out,
                        int64_t rows, int64_t cols, void* stream, bool quant) {
  if (rows < 0 || cols <= 0) return mxq_set_error(MXQ_ERR_INVALID, "bad shape");
  if (rows == 0) return MXQ_OK;
  if (!x || !scale || !shift) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  if (scale_group <= 0 || shift_group <= 0)
    return mxq_set_error(MXQ_ERR_INVALID, "modulation groups must be positive");
  if (quant && (!q || !scales)) return mxq_set_error(MXQ_ERR_INVALID, "null output");
  const int nch = pick_nch(cols);
  if (cols % 8 != 0 || nch == 0 || nch > 16 || (uintptr_t)x % 16 || (uintptr_t)scale % 16 ||
      (uintptr_t)shift % 16 || (y_out && (uintptr_t)y_out % 16) || (q && (uintptr_t)q % 8))
    return mxq_set_error(MXQ_ERR_UNSUPPORTED,
                         "adaLN needs cols %% 8 == 0, cols <= 8192 and 16-byte aligned rows");
  hipStream_t st = (hipStream_t)stream;
  const int64_t need = (cols / 8 + kWave - 1) / kWave;
  const int uch = need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : need <= 6 ? 6 : need <= 8 ? 8 : need <= 10 ? 10
                : need <= 11 ? 11 : need <= 12 ? 12 : need <= 14 ? 14 : 16;
  if (scale_group >= rows && shift_group >= rows && cols <= kAdalnMaxCols && (cols == uch * 512 || uch <= 12)) {
    // one modulation row: the two-buffer kernel (widths whose register budget it fits)
    // Every workgroup takes an equal share of the rows, so the grid is what fits on the device at
    // once: a larger one left its last workgroups to start after the first had finished.
    const size_t lds = (size_t)cols * 2 * sizeof(float);
    const int64_t wg = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
#define MXQ_ADALN_UNIFORM_K(N_, E_)                                                                              \
  (quant ? (void)(adaln_uniform_rows<N_, true, E_><<<mxq_resident_grid(adaln_uniform_rows<N_, true, E_>,          \
                                                                       kQuantBlock, lds, wg),                    \
                                                     kQuantBlock, lds, st>>>(                                    \
               (const uint16_t*)x, (const uint16_t*)scale, (const uint16_t*)shift, eps, q, scales,              \
               (uint16_t*)y_out, rows, (int)cols))                                                               \
         : (void)(adaln_uniform_rows<N_, false, E_><<<mxq_resident_grid(adaln_uniform_rows<N_, false, E_>,        \
                                                                        kQuantBlock, lds, wg),                   \
                                                      kQuantBlock, lds, st>>>(                                   \
               (const uint16_t*)x, (const uint16_t*)scale, (const uint16_t*)shift, eps, nullptr, nullptr,        \
               (uint16_t*)y_out, rows, (int)cols)))
#define MXQ_ADALN_UNIFORM(N_) \
  (cols == (N_) * 512 ? MXQ_ADALN_UNIFORM_K(N_, true) : MXQ_ADALN_UNIFORM_K(N_, false))
    switch (uch) {
      case 1: MXQ_ADALN_UNIFORM(1); break;
      case 2: MXQ_ADALN_UNIFORM(2); break;
      case 4: MXQ_ADALN_UNIFORM(4); break;
      case 6: MXQ_ADALN_UNIFORM(6); break;
      case 8: MXQ_ADALN_UNIFORM(8); break;
      case 10: MXQ_ADALN_UNIFORM(10); break;
      case 11: MXQ_ADALN_UNIFORM(11); break;
      case 12: MXQ_ADALN_UNIFORM(12); break;
      case 14: MXQ_ADALN_UNIFORM(14); break;
      default: MXQ_ADALN_UNIFORM(16); break;
    }
#undef MXQ_ADALN_UNIFORM
#undef MXQ_ADALN_UNIFORM_K
    return mxq_check_launch("adaln_uniform_rows");
  }
  if (quant) {
    MXQ_NCH_SWITCH_16(nch, (adaln_rows_reg<N_, true><<<adaln_grid(rows), kQuantBlock, 0, st>>>(
                             (const uint16_t*)x, (const uint16_t*)scale, (const uint16_t*)shift,
                             scale_group, shift_group, eps, q, scales, (uint16_t*)y_out, rows,
                             (int)cols)));
  } else {
    MXQ_NCH_SWITCH_16(nch, (adaln_rows_reg<N_, false><<<adaln_grid(rows), kQuantBlock, 0, st>>>(
                             (const uint16_t*)x, (const uint16_t*)scale, (const uint16_t*)shift,
                             scale_group, shift_group, eps, nullptr, nullptr, (uint16_t*)y_out,
                             rows, (int)cols)));
  }
  return mxq_check_launch("adaln_rows_reg");
}

extern "C" int mxq_adaln(const void* x, const void* scale, const void* shift, void* out,
                         int64_t rows, int64_t cols, int64_t scale_group, int64_t shift_group,
                         float eps, void* stream) {
  if (!out) return mxq_set_error(MXQ_ERR_INVALID, "null output");
  return adaln_launch(x, scale, shift, scale_group, shift_group, eps, nullptr, nullptr, out, rows,
                      cols, stream, false);
}

extern "C" int mxq_adaln_quantize_int8(const void* x, const void* scale, const void* shift,
                                       int64_t scale_group, int64_t shift_group, float eps,
                                       int8_t* q, float* scales, void* y_out, int64_t rows,
                                       int64_t cols, void* stream) {
  return adaln_launch(x, scale, shift, scale_group, shift_group, eps, q, scales, y_out, rows, cols,
                      stream, true);
}

extern "C" int mxq_fill_f32(float* p, float value, int64_t n, void* stream) {
  if (n < 0) return mxq_set_error(MXQ_ERR_INVALID, "negative length");
  if (n == 0) return MXQ_OK;
  if (!p) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  fill_f32_kernel<<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>(p, value, n);
  return mxq_check_launch("fill_f32");
}

extern "C" int mxq_gelu_tanh_bf16(const void* x, void* y, int64_t n, void* stream) {
  if (n < 0) return mxq_set_error(MXQ_ERR_INVALID, "negative length");
  if (n == 0) return MXQ_OK;
  if (!x || !y) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  const int vec = ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % 16 == 0);
  int64_t blocks = (n / 8 + 255) / 256 + 1;
  if (blocks > 65536) blocks = 65536;
  gelu_bf16_kernel<<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>((const uint16_t*)x, (uint16_t*)y, n, vec);
  return mxq_check_launch("gelu_bf16_kernel");
}

extern "C" int mxq_input_act_f16(const void* x, void* y, int64_t rows, int64_t cols, int input_act, void* stream) {
  if (rows < 0 || cols < 0) return mxq_set_error(MXQ_ERR_INVALID, "negative shape");
  if (input_act != MXQ_ACT_GELU_TANH && input_act != MXQ_ACT_SWIGLU)
    return mxq_set_error(MXQ_ERR_INVALID, "unsupported input_act code %d", input_act);
  if (rows == 0 || cols == 0) return MXQ_OK;
  if (!x || !y) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  if (rows > INT64_MAX / 2 / cols) return mxq_set_error(MXQ_ERR_INVALID, "shape too large");
  const int64_t blocks = std::min<int64_t>((rows * cols + 255) / 256, 65536);
  hipStream_t st = (hipStream_t)stream;
  if (input_act == MXQ_ACT_GELU_TANH)
    act_f16_kernel<MXQ_ACT_GELU_TANH><<<(unsigned)blocks, 256, 0, st>>>((const uint16_t*)x, (uint16_t*)y, rows, cols);
  else
    act_f16_kernel<MXQ_ACT_SWIGLU><<<(unsigned)blocks, 256, 0, st>>>((const uint16_t*)x, (uint16_t*)y, rows, cols);
  return mxq_check_launch("act_f16_kernel");
}

extern "C" int mxq_adaln_quantize_int8_f16(const void* x, const void* scale, const void* shift,
                                           int64_t scale_group, int64_t shift_group, float eps, int8_t* q,
                                           float* scales, void* y_out, int64_t rows, int64_t cols, void* stream) {
  if (rows < 0 || cols <= 0) return mxq_set_error(MXQ_ERR_INVALID, "bad shape");
  if (rows == 0) return MXQ_OK;
  if (!x || !scale || !shift) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  if (scale_group <= 0 || shift_group <= 0) return mxq_set_error(MXQ_ERR_INVALID, "modulation groups must be positive");
  if (!q != !scales) return mxq_set_error(MXQ_ERR_INVALID, "q and scales go together");
  if (!q && !y_out) return mxq_set_error(MXQ_ERR_INVALID, "neither a modulated output nor a quantized output");
  adaln_f16_rows<<<row_grid(rows), kQuantBlock, 0, (hipStream_t)stream>>>(
      (const uint16_t*)x, (const uint16_t*)scale, (const uint16_t*)shift, scale_group, shift_group, eps, q, scales,
      (uint16_t*)y_out, rows, cols);
  return mxq_check_launch("adaln_f16_rows");
}
