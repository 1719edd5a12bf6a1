// Offline W4A8 weight preparation on gfx950: ConvRot rotation of the weight rows and the
// reference's grouped int4 storage (codes, relative group scales, channel scales, and for the
// asymmetric mode the correction term), the load-time counterpart of
// backends/turbo/vendor/comfy_kitchen/backends/eager/w4a8_int8.py:122-209, 315-341 (CK below).
//
// One 256-thread workgroup per weight row (K <= 16384: the row is held in LDS as float64).
//  1. Rotation (ConvRot group cg, a power of 4, or none): the radix-4 transform of the activation
//     quantizers in the same operation order (digits 0-3: y_k = S - 2 x_{3-k}, S = (x0 + x1) +
//     (x2 + x3); digits >= 4: (x_k + x_{k^1}) + (x_{k^2} - x_{k^3})), then the 2^-d factor and
//     one rounding to the weight's dtype: the exact product W_grouped @ H^T rounded once.
//  2. Per group of G weights, in float32 (CK/backends/eager/w4a8_int8.py:150-187):
//       codebook mode: s = max |w| (>= 1e-8), codes by nearest level of w / s, three refinements
//         s = (sum w * cb[c]) / (sum cb[c]^2) (each >= 1e-8), codes re-assigned after each;
//       symmetric mode: s = max(max |w| / 7, 1e-8), c = clamp(rne(w / s), -8, 7) + 8;
//       asymmetric mode: s = max((max w - min w) / 15, 1e-8), c = clamp(rne((w - min) / s), 0, 15),
//         correction = dtype(8 s + min);
//     the row's s_channel = max(max over groups of |shifted value| / 127, 1e-8) (block reduction).
//  3. s_rel = s / s_channel (float32, or float8_e4m3fn: round to nearest even, beyond the format
//     NaN, as torch converts), and in the codebook mode the final codes by the nearest decoded
//     level clamp(rne(cb * s_rel), +-127) to w / s_channel; codes packed two per byte, even k in
//     the low nibble (CK/backends/eager/w4a8_int8.py:200-202).
// Group sums of <= 32 terms use torch's CPU order for a last-dimension reduction (eight
// interleaved partial sums added in order; fewer than eight terms in order); nearest-level
// searches keep the first level on ties (strict <, CK/backends/eager/w4a8_int8.py:35-63).

#include "act_rot.h"

namespace mxq {

namespace {

constexpr int kQThreads = 256;
constexpr int kQMaxK = 16384;
constexpr int kQMinGroup = 4;

enum { kW4Codebook = 0, kW4Symmetric = 1, kW4Asymmetric = 2, kW4RotateOnly = 3 };

struct W4QArgs {
  const void* w;
  int64_t N, K;
  int G, cg_digits, mode, w_bf16, srel_e4m3;
  const float* codebook;
  int8_t* packed;
  void* s_rel;
  float* s_channel;
  void* correction;
  void* rotated;
};

MXQ_DEVICE float e4m3fn_value(uint32_t b) {
  const uint32_t e = (b >> 3) & 0xFu, m = b & 7u;
  if ((b & 0x7Fu) == 0x7Fu) return __uint_as_float(0x7FC00000u);
  const float v = e == 0 ? (float)m * 0.001953125f : __uint_as_float(((e + 120u) << 23) | (m << 20));
  return (b & 0x80u) ? -v : v;
}

// float32 -> float8_e4m3fn bits: the 3-bit significand rounded to nearest even from the float32
// bits (a carry moves into the exponent), values below 2^-6 on the subnormal grid of 2^-9;
// magnitudes that round beyond 448 (above 464) give the NaN code 0x7F.
MXQ_DEVICE uint32_t e4m3fn_bits(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7FFFFFFFu;
  uint32_t b;
  if (a > 0x7F800000u) {
    b = 0x7Fu;
  } else if (a < 0x3C800000u) {  // below 2^-6
    b = (uint32_t)__builtin_rintf(__uint_as_float(a) * 512.0f);
  } else {
    const uint32_t r = (a + 0x7FFFFu + ((a >> 20) & 1u)) >> 20;
    b = r - 960u < 0x7Fu ? r - 960u : 0x7Fu;
  }
  return sign | b;
}

// Index of the nearest of 16 levels (first on ties).
MXQ_DEVICE int nearest16(float v, const float* lv) {
  float best = fabsf(v - lv[0]);
  int idx = 0;
#pragma unroll
  for (int i = 1; i < 16; ++i) {
    const float d = fabsf(v - lv[i]);
    if (d < best) {
      best = d;
      idx = i;
    }
  }
  return idx;
}

// Running sum in torch's CPU order for n <= 32 terms (term i into partial i % 8 when n >= 8).
struct Sum8 {
  float p[8];
  int n;
  MXQ_DEVICE void init(int terms) {
    n = terms;
#pragma unroll
    for (int j = 0; j < 8; ++j) p[j] = 0.0f;
  }
  MXQ_DEVICE void add(int i, float v) {
    if (n < 8) {
      p[0] = i == 0 ? v : p[0] + v;
    } else {
      const int j = i & 7;
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (q == j) p[q] = i < 8 ? v : p[q] + v;
    }
  }
  MXQ_DEVICE float total() const {
    if (n < 8) return p[0];
    float s = p[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) s = s + p[j];
    return s;
  }
};

__global__ __launch_bounds__(kQThreads) void w4a8_quant_rows(W4QArgs p) {
  __shared__ double s_row[kQMaxK];
  __shared__ float s_gs[kQMaxK / kQMinGroup];
  __shared__ float s_cb[16];
  __shared__ float s_red[kQThreads / kWave];
  const int t = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int K = (int)p.K, G = p.G, groups = K / G;
  if (t < 16) s_cb[t] = p.codebook ? p.codebook[t] : 0.0f;
  for (int c = t; c < K; c += kQThreads) {
    s_row[c] = p.w_bf16 ? (double)bf16_to_f32(reinterpret_cast<const uint16_t*>(p.w)[row * K + c])
                        : (double)reinterpret_cast<const float*>(p.w)[row * K + c];
  }
  __syncthreads();

  // ---- 1. rotation
  if (p.cg_digits > 0) {
    const int cg = 1 << (2 * p.cg_digits);
    for (int d = 0; d < p.cg_digits; ++d) {
      const int stride = 1 << (2 * d);
      for (int q = t; q < K / 4; q += kQThreads) {
        const int group = q / (cg / 4), r = q - group * (cg / 4);
        const int low = r % stride, high = r / stride;
        const int base = group * cg + high * stride * 4 + low;
        double x0 = s_row[base], x1 = s_row[base + stride], x2 = s_row[base + 2 * stride], x3 = s_row[base + 3 * stride];
        if (d < 4) {
          h4_quad(x0, x1, x2, x3);
        } else {
          const double y0 = (x0 + x1) + (x2 - x3), y1 = (x1 + x0) + (x3 - x2);
          const double y2 = (x2 + x3) + (x0 - x1), y3 = (x3 + x2) + (x1 - x0);
          x0 = y0;
          x1 = y1;
          x2 = y2;
          x3 = y3;
        }
        s_row[base] = x0;
        s_row[base + stride] = x1;
        s_row[base + 2 * stride] = x2;
        s_row[base + 3 * stride] = x3;
      }
      __syncthreads();
    }
    const double inv = 1.0 / (double)(1 << p.cg_digits);
    for (int c = t; c < K; c += kQThreads) {
      const double v = s_row[c] * inv;
      if (p.w_bf16) {
        const uint32_t b = f64_to_bf16_bits(v);
        s_row[c] = (double)bf16_to_f32(b);
        if (p.rotated) reinterpret_cast<uint16_t*>(p.rotated)[row * K + c] = (uint16_t)b;
      } else {
        const float f = (float)v;
        s_row[c] = (double)f;
        if (p.rotated) reinterpret_cast<float*>(p.rotated)[row * K + c] = f;
      }
    }
    __syncthreads();
  }
  if (p.mode == kW4RotateOnly) return;

  // ---- 2. group scales and the row's channel scale
  auto w_at = [&](int g, int i) { return (float)s_row[g * G + i]; };
  float tmax = 0.0f;
  for (int g = t; g < groups; g += kQThreads) {
    float s, shifted = 0.0f;
    if (p.mode == kW4Codebook) {
      float amax = 0.0f;
      for (int i = 0; i < G; ++i) amax = fmaxf(amax, fabsf(w_at(g, i)));
      s = fmaxf(amax, 1e-8f);
      for (int it = 0; it < 3; ++it) {  // codes from s, then the least-squares scale
        Sum8 num, den;
        num.init(G);
        den.init(G);
        for (int i = 0; i < G; ++i) {
          const float w = w_at(g, i);
          const float qc = s_cb[nearest16(w / s, s_cb)];
          num.add(i, w * qc);
          den.add(i, qc * qc);
        }
        s = fmaxf(num.total() / fmaxf(den.total(), 1e-8f), 1e-8f);
      }
      for (int i = 0; i < G; ++i) shifted = fmaxf(shifted, fabsf(s_cb[nearest16(w_at(g, i) / s, s_cb)] * s));
    } else if (p.mode == kW4Symmetric) {
      float amax = 0.0f;
      for (int i = 0; i < G; ++i) amax = fmaxf(amax, fabsf(w_at(g, i)));
      s = fmaxf(amax / 7.0f, 1e-8f);
      for (int i = 0; i < G; ++i) {
        const float v = fminf(fmaxf(__builtin_rintf(w_at(g, i) / s), -8.0f), 7.0f);
        shifted = fmaxf(shifted, fabsf(v * s));
      }
    } else {
      float mn = w_at(g, 0), mx = mn;
      for (int i = 1; i < G; ++i) {
        mn = fminf(mn, w_at(g, i));
        mx = fmaxf(mx, w_at(g, i));
      }
      s = fmaxf((mx - mn) / 15.0f, 1e-8f);
      for (int i = 0; i < G; ++i) {
        const float c = fminf(fmaxf(__builtin_rintf((w_at(g, i) - mn) / s), 0.0f), 15.0f);
        shifted = fmaxf(shifted, fabsf((c - 8.0f) * s));
      }
    }
    s_gs[g] = s;
    tmax = fmaxf(tmax, shifted);
  }
  // block maximum (non-negative values: the float order is the bit order)
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, o, kWave));
  if ((t & (kWave - 1)) == 0) s_red[t / kWave] = tmax;
  __syncthreads();
  float rmax = s_red[0];
#pragma unroll
  for (int i = 1; i < kQThreads / kWave; ++i) rmax = fmaxf(rmax, s_red[i]);
  const float s_ch = fmaxf(rmax / 127.0f, 1e-8f);
  if (t == 0) p.s_channel[row] = s_ch;

  // ---- 3. relative scales, final codes, packing
  uint8_t* out = reinterpret_cast<uint8_t*>(p.packed) + row * (K / 2);
  for (int g = t; g < groups; g += kQThreads) {
    const float s = s_gs[g];
    float srel = s / s_ch;
    if (p.srel_e4m3) {
      const uint32_t b = e4m3fn_bits(srel);
      reinterpret_cast<uint8_t*>(p.s_rel)[row * groups + g] = (uint8_t)b;
      srel = e4m3fn_value(b);
    } else {
      reinterpret_cast<float*>(p.s_rel)[row * groups + g] = srel;
    }
    float lv[16];
    float mn = 0.0f;
    if (p.mode == kW4Codebook) {
#pragma unroll
      for (int i = 0; i < 16; ++i) lv[i] = fminf(fmaxf(__builtin_rintf(s_cb[i] * srel), -127.0f), 127.0f);
    } else if (p.mode == kW4Asymmetric) {
      mn = w_at(g, 0);
      for (int i = 1; i < G; ++i) mn = fminf(mn, w_at(g, i));
      const float corr = 8.0f * s + mn;
      if (p.w_bf16)
        reinterpret_cast<uint16_t*>(p.correction)[(int64_t)g * p.N + row] = (uint16_t)f32_to_bf16_bits(corr);
      else
        reinterpret_cast<float*>(p.correction)[(int64_t)g * p.N + row] = corr;
    }
    for (int i = 0; i < G; i += 2) {
      uint32_t c[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float w = w_at(g, i + h);
        if (p.mode == kW4Codebook)
          c[h] = (uint32_t)nearest16(w / s_ch, lv);
        else if (p.mode == kW4Symmetric)
          c[h] = (uint32_t)((int)fminf(fmaxf(__builtin_rintf(w / s), -8.0f), 7.0f) + 8);
        else
          c[h] = (uint32_t)fminf(fmaxf(__builtin_rintf((w - mn) / s), 0.0f), 15.0f);
      }
      out[(g * G + i) / 2] = (uint8_t)((c[0] & 0xFu) | ((c[1] & 0xFu) << 4));
    }
  }
}

}  // namespace

}  // namespace mxq

using namespace mxq;

extern "C" int mxq_w4a8_quantize_weight(const void* w, int w_dtype, int64_t N, int64_t K, int64_t group_size,
                                        int64_t convrot_groupsize, int mode, const float* codebook,
                                        int s_rel_dtype, int8_t* packed, void* s_rel, float* s_channel,
                                        void* correction, void* rotated_out, void* stream) {
  if (N < 0 || K < 0) return mxq_set_error(MXQ_ERR_INVALID, "negative shape");
  const int64_t G = group_size, cg = convrot_groupsize;
  if (mode < 0 || mode > 3) return mxq_set_error(MXQ_ERR_INVALID, "unknown W4A8 storage mode %d", mode);
  if (K % 16 != 0 || G < 4 || (16 % G != 0 && G % 16 != 0) || K % G != 0 || (cg > 0 && K % cg != 0))
    return mxq_set_error(MXQ_ERR_INVALID,
                         "K=%lld must be divisible by 16, group_size=%lld, and convrot_groupsize=%lld; "
                         "group_size must be >=4 and divide 16 or be a multiple of 16",
                         (long long)K, (long long)G, (long long)cg);
  int digits = 0;
  if (cg > 0) {
    if (cg < 4 || (cg & (cg - 1)) || ((__builtin_ctzll(cg)) & 1))
      return mxq_set_error(MXQ_ERR_INVALID, "Regular Hadamard size must be a power of 4, got %lld", (long long)cg);
    digits = __builtin_ctzll(cg) / 2;
  }
  if (K > kQMaxK || G > 128)
    return mxq_set_error(MXQ_ERR_UNSUPPORTED, "weight preparation takes K <= %d and group_size <= 128", kQMaxK);
  if (w_dtype != MXQ_DTYPE_BF16 && w_dtype != MXQ_DTYPE_F32)
    return mxq_set_error(MXQ_ERR_UNSUPPORTED, "weight dtype code %d (bf16 or fp32)", w_dtype);
  if (s_rel_dtype != MXQ_DTYPE_F32 && s_rel_dtype != MXQ_DTYPE_E4M3)
    return mxq_set_error(MXQ_ERR_UNSUPPORTED, "s_rel dtype code %d", s_rel_dtype);
  if (N == 0 || K == 0) return MXQ_OK;
  if (!w) return mxq_set_error(MXQ_ERR_INVALID, "null weight");
  if (mode == kW4RotateOnly) {
    if (!rotated_out || digits == 0) return mxq_set_error(MXQ_ERR_INVALID, "rotation only needs a group and an output");
  } else {
    if (!packed || !s_rel || !s_channel) return mxq_set_error(MXQ_ERR_INVALID, "null output");
    if (mode == kW4Codebook && !codebook) return mxq_set_error(MXQ_ERR_INVALID, "the codebook mode needs a codebook");
    if (mode == kW4Asymmetric && !correction) return mxq_set_error(MXQ_ERR_INVALID, "the asymmetric mode needs a correction output");
  }
  if (N > INT32_MAX) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "too many rows");
  W4QArgs a{};
  a.w = w;
  a.N = N;
  a.K = K;
  a.G = (int)G;
  a.cg_digits = digits;
  a.mode = mode;
  a.w_bf16 = w_dtype == MXQ_DTYPE_BF16;
  a.srel_e4m3 = s_rel_dtype == MXQ_DTYPE_E4M3;
  a.codebook = codebook;
  a.packed = packed;
  a.s_rel = s_rel;
  a.s_channel = s_channel;
  a.correction = correction;
  a.rotated = rotated_out;
  w4a8_quant_rows<<<(unsigned)N, kQThreads, 0, (hipStream_t)stream>>>(a);
  return mxq_check_launch("w4a8_quant_rows");
}
