// M = 1 INT8 linear (gfx950): the per-token quantizer -- with the optional input activation and
// ConvRot rotation -- fused with the INT8 GEMV and the dequant epilogue, in one launch.
//
// Reference: int8_linear's M = 1 route (backends/turbo/vendor/comfy_kitchen/backends/cuda/
// __init__.py:1999-2034) and its fused quantize + GEMV kernels (CK/backends/cuda/ops/
// int8_linear.cu:411-492, 1490-1590). Values follow the eager composition instead
// (CK/backends/eager/quantization.py:971-1056: the row quantizer, the int8 matmul, then
// y = out(fp32(acc) * (xs * ws)), y = out(y + bias)), so a token gives the same bits whether
// it is alone or part of a batch; the reference's CUDA GEMV multiplies the scales in another
// order and adds the bias before its single rounding.
//
// Layout: 512-thread blocks, one output column per wave (eight per block). Each wave first
// issues the loads of its weight row (16 bytes per lane per 1024 columns, K <= 16384), so the
// row is in flight while the block quantizes x into LDS: each wave takes one 1024-column window
// per pass (lane l: columns 16 l .. 16 l + 15, the ConvRot layout), the absmax is reduced through
// LDS, and the int8 row is written to LDS. Then every wave forms its dot product with v_dot4,
// reduces it across the wave and lane 0 applies the epilogue. Each block quantizes x itself:
// the row is at most 32 KB and stays in L2, and the redundant work overlaps the weight stream.

#include "act_rot.h"

namespace mxq {
namespace {

constexpr int kM1Waves = 8;
constexpr int kM1Threads = kM1Waves * kWave;
constexpr int kM1MaxChunks = 16;                    // 16-byte weight chunks per lane
constexpr int kM1MaxK = kM1MaxChunks * kWave * 16;  // 16384

struct M1Args {
  const uint16_t* x;  // bf16 row [K] ([2K] for SwiGLU), when the kernel quantizes
  const int8_t* xq;   // int8 row [K] and its scale, when already quantized
  const float* xs;
  const int8_t* w;    // [N, K]
  const float* ws;    // [1] or [N]
  const void* bias;   // [N] in the output dtype, or null
  void* out;          // [N]
  int8_t* xq_out;     // optional: the quantized row and its scale (written by block 0)
  float* xs_out;
  int64_t N;
  int K, digits, ws_per_channel;
};

MXQ_DEVICE int wave_sum_i32(int v) {
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

template <int kAct, int kOut, bool kQuant>
__global__ __launch_bounds__(kM1Threads) void linear_m1_kernel(M1Args p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * kM1Waves + wave;
  const bool col_on = n < p.N;
  const int chunks = p.K >> 4;

  // ---- the weight row of this wave, in flight during the quantizer
  const int8_t* wr = p.w + (col_on ? n : 0) * (int64_t)p.K;
  v4i wv[kM1MaxChunks];
#pragma unroll
  for (int j = 0; j < kM1MaxChunks; ++j) {
    const int c = j * kWave + lane;
    wv[j] = (col_on && c < chunks) ? *reinterpret_cast<const v4i*>(wr + (int64_t)c * 16) : v4i{0, 0, 0, 0};
  }

  // ---- the quantized activation row
  const int8_t* xq;
  float s;
  if constexpr (kQuant) {
    uint16_t* rowbuf = reinterpret_cast<uint16_t*>(smem);         // rotated bf16 row [K]
    int8_t* xql = reinterpret_cast<int8_t*>(smem + 2 * p.K);       // int8 row [K]
    float* red = reinterpret_cast<float*>(smem + 3 * p.K);         // wave maxima [kM1Waves]
    const double inv = 1.0 / (double)(1 << p.digits);
    float amax = 0.0f;
    for (int base = 0; base < p.K; base += kM1Waves * 1024) {
      const int e0 = base + wave * 1024 + lane * 16;
      const bool on = e0 < p.K;
      double v[16];
      load16_act<kAct>(p.x, p.K, e0, on, v);
      rotate16(v, p.digits);  // groups never straddle K (K % G == 0): lanes past K hold zeros
      if (on) {
        uint32_t h[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t lo = f64_to_bf16_bits(v[2 * i] * inv), hi = f64_to_bf16_bits(v[2 * i + 1] * inv);
          h[i] = lo | (hi << 16);
          amax = fmaxf(amax, fmaxf(fabsf(bf16_to_f32(lo)), fabsf(bf16_to_f32(hi))));
        }
        v4u* dst = reinterpret_cast<v4u*>(rowbuf + e0);
        dst[0] = v4u{h[0], h[1], h[2], h[3]};
        dst[1] = v4u{h[4], h[5], h[6], h[7]};
      }
    }
    amax = wave_max(amax);
    if (lane == 0) red[wave] = amax;
    __syncthreads();
    amax = red[0];
#pragma unroll
    for (int i = 1; i < kM1Waves; ++i) amax = fmaxf(amax, red[i]);
    s = row_scale_from_absmax(amax);
    const float r = 1.0f / round_bf16(s);
    for (int base = 0; base < p.K; base += kM1Waves * 1024) {
      const int e0 = base + wave * 1024 + lane * 16;
      if (e0 >= p.K) continue;
      const v4u* src = reinterpret_cast<const v4u*>(rowbuf + e0);  // written by this lane
      uint32_t o[4];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const v4u w = src[c];
        int qv[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          qv[2 * i] = quant_round_clamp(round_bf16(bf16_to_f32(w[i] & 0xFFFFu) * r));
          qv[2 * i + 1] = quant_round_clamp(round_bf16(bf16_to_f32(w[i] >> 16) * r));
        }
        o[2 * c] = (uint32_t)(qv[0] & 0xFF) | ((uint32_t)(qv[1] & 0xFF) << 8) | ((uint32_t)(qv[2] & 0xFF) << 16) |
                   ((uint32_t)(qv[3] & 0xFF) << 24);
        o[2 * c + 1] = (uint32_t)(qv[4] & 0xFF) | ((uint32_t)(qv[5] & 0xFF) << 8) |
                       ((uint32_t)(qv[6] & 0xFF) << 16) | ((uint32_t)(qv[7] & 0xFF) << 24);
      }
      *reinterpret_cast<v4u*>(xql + e0) = v4u{o[0], o[1], o[2], o[3]};
      if (blockIdx.x == 0 && p.xq_out) *reinterpret_cast<v4u*>(p.xq_out + e0) = v4u{o[0], o[1], o[2], o[3]};
    }
    if (blockIdx.x == 0 && threadIdx.x == 0 && p.xs_out) p.xs_out[0] = s;
    __syncthreads();
    xq = xql;
  } else {
    xq = p.xq;
    s = p.xs[0];
  }

  // ---- dot product, wave reduction, epilogue
  int acc = 0;
#pragma unroll
  for (int j = 0; j < kM1MaxChunks; ++j) {
    const int c = j * kWave + lane;
    if (c < chunks) {
      const v4i xv = *reinterpret_cast<const v4i*>(xq + (int64_t)c * 16);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_sdot4(xv[e], wv[j][e], acc, false);
    }
  }
  acc = wave_sum_i32(acc);
  if (lane == 0 && col_on) {
    typedef typename OutT<kOut>::T T;
    const float wsn = p.ws[p.ws_per_channel ? n : 0];
    const float b = p.bias ? OutT<kOut>::load(reinterpret_cast<const T*>(p.bias) + n) : -0.0f;
    const float y = OutT<kOut>::round((float)acc * (s * wsn));
    store_out<kOut>(reinterpret_cast<T*>(p.out) + n, y + b);
  }
}

template <int kAct, bool kQuant>
int launch_m1(const M1Args& a, int out_dtype, hipStream_t st) {
  const unsigned grid = (unsigned)((a.N + kM1Waves - 1) / kM1Waves);
  const size_t lds = kQuant ? (size_t)3 * a.K + 16 * kM1Waves : 0;
  switch (out_dtype) {
    case MXQ_DTYPE_F32: linear_m1_kernel<kAct, 0, kQuant><<<grid, kM1Threads, lds, st>>>(a); break;
    case MXQ_DTYPE_F16: linear_m1_kernel<kAct, 1, kQuant><<<grid, kM1Threads, lds, st>>>(a); break;
    case MXQ_DTYPE_BF16: linear_m1_kernel<kAct, 2, kQuant><<<grid, kM1Threads, lds, st>>>(a); break;
    default: return mxq_set_error(MXQ_ERR_UNSUPPORTED, "output dtype code %d", out_dtype);
  }
  return mxq_check_launch("linear_m1_kernel");
}

int check_m1(const void* x, const int8_t* w, const float* ws, int64_t ws_numel, void* out, int64_t N,
             int64_t K) {
  if (N < 0 || K < 0) return mxq_set_error(MXQ_ERR_INVALID, "negative shape");
  if (N == 0) return MXQ_OK;
  if (!x || !w || !ws || !out) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  if (ws_numel != 1 && ws_numel != N)
    return mxq_set_error(MXQ_ERR_INVALID, "weight scale must have 1 or N=%lld entries, got %lld", (long long)N,
                         (long long)ws_numel);
  if (K == 0 || K % 16 || K > kM1MaxK)
    return mxq_set_error(MXQ_ERR_UNSUPPORTED, "M = 1 path needs K a multiple of 16 in [16, %d], got %lld", kM1MaxK,
                         (long long)K);
  if ((uintptr_t)x % 16 || (uintptr_t)w % 16) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "x and w must be 16-byte aligned");
  if (N > (int64_t)kM1Waves * 0x7FFFFFFF) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "N too large");
  return MXQ_OK;
}

}  // namespace
}  // namespace mxq

using namespace mxq;

extern "C" int mxq_int8_linear_m1(const void* x_bf16, const int8_t* w, const float* ws, int64_t ws_numel,
                                  const void* bias, void* out, int64_t N, int64_t K, int64_t group_size,
                                  int input_act, int out_dtype, int8_t* xq_out, float* xs_out, void* stream) {
  int rc = check_m1(x_bf16, w, ws, ws_numel, out, N, K);
  if (rc || N == 0) return rc;
  int digits = 0;
  if (group_size != 0) {
    if (group_size < 4 || (group_size & (group_size - 1)) || __builtin_ctzll((uint64_t)group_size) % 2)
      return mxq_set_error(MXQ_ERR_INVALID, "Regular Hadamard size must be a power of 4, got %lld", (long long)group_size);
    if (K % group_size)
      return mxq_set_error(MXQ_ERR_INVALID, "ConvRot group size %lld does not divide input features %lld",
                           (long long)group_size, (long long)K);
    if (group_size > 1024) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "ConvRot group size above 1024");
    digits = __builtin_ctzll((uint64_t)group_size) / 2;
  }
  if ((uintptr_t)xq_out % 16) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "xq_out must be 16-byte aligned");
  M1Args a{};
  a.x = (const uint16_t*)x_bf16; a.w = w; a.ws = ws; a.bias = bias; a.out = out;
  a.xq_out = xq_out; a.xs_out = xs_out;
  a.N = N; a.K = (int)K; a.digits = digits; a.ws_per_channel = ws_numel == N && N != 1;
  hipStream_t st = (hipStream_t)stream;
  switch (input_act) {
    case MXQ_ACT_NONE: return launch_m1<MXQ_ACT_NONE, true>(a, out_dtype, st);
    case MXQ_ACT_GELU_TANH: return launch_m1<MXQ_ACT_GELU_TANH, true>(a, out_dtype, st);
    case MXQ_ACT_SWIGLU: return launch_m1<MXQ_ACT_SWIGLU, true>(a, out_dtype, st);
    default: return mxq_set_error(MXQ_ERR_INVALID, "unsupported input_act code %d", input_act);
  }
}

extern "C" int mxq_int8_gemv_dequant(const int8_t* xq, const float* xs, const int8_t* w, const float* ws,
                                     int64_t ws_numel, const void* bias, void* out, int64_t N, int64_t K,
                                     int out_dtype, void* stream) {
  int rc = check_m1(xq, w, ws, ws_numel, out, N, K);
  if (rc || N == 0) return rc;
  if (!xs) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  M1Args a{};
  a.xq = xq; a.xs = xs; a.w = w; a.ws = ws; a.bias = bias; a.out = out;
  a.N = N; a.K = (int)K; a.ws_per_channel = ws_numel == N && N != 1;
  return launch_m1<MXQ_ACT_NONE, false>(a, out_dtype, (hipStream_t)stream);
}
