// M = 1 INT8 linear (gfx950): the per-token quantizer (with the optional input activation and
// ConvRot rotation) followed by a weight-streaming INT8 GEMV with the dequant epilogue.
//
// Reference: int8_linear's M = 1 route (backends/turbo/vendor/comfy_kitchen/backends/cuda/
// __init__.py:1999-2034) and its GEMV kernels (CK/backends/cuda/ops/int8_linear.cu:411-492,
// 1490-1590). Values follow the eager composition instead (CK/backends/eager/quantization.py:
// 971-1056: the row quantizer, the int8 matmul, then y = out(fp32(acc) * (xs * ws)),
// y = out(y + bias)), so a token gives the same bits whether it is alone or part of a batch;
// the reference's CUDA GEMV multiplies the scales in another order and adds the bias before its
// single rounding.
//
// The quantizer is the row kernel of mxq_quantize_int8_rowwise_convrot (one row: a single
// workgroup). The GEMV is bound by streaming the [N, K] weights once: each wave owns kCols
// output columns, issues all their 16-byte loads (lane l takes chunks l, l + 64, ... of a row,
// so every load instruction reads 1 KB of contiguous weights; nontemporal, as the weights are
// read once per token: 5376 x 21504 cycled through four layers 20.9 -> 19.3 us) before the
// first use, forms the dot products with v_dot4 against the quantized row (read once per wave,
// L2-resident), reduces them across the wave and applies the epilogue. A launch is sized by K (chunks per lane) and
// N (one or two columns per wave), so that many waves each keep a few KB of weights in flight.

#include "mxq_common.h"

extern "C" int mxq_quantize_int8_rowwise_convrot(const void* x, int x_dtype, int8_t* q, float* scales,
                                                 int64_t rows, int64_t cols, int64_t group_size,
                                                 int input_act, void* stream);

namespace mxq {
namespace {

constexpr int kGvWaves = 4;
constexpr int kGvThreads = kGvWaves * kWave;
constexpr int kGvMaxK = 16384;  // 16 chunks of 16 bytes per lane

struct GvArgs {
  const int8_t* xq;   // int8 row [K]
  const float* xs;    // its scale [1]
  const int8_t* w;    // [N, K]
  const float* ws;    // [1] or [N]
  const void* bias;   // [N] in the output dtype, or null
  void* out;          // [N]
  int64_t N;
  int K, ws_per_channel;
};

// kChunks: 16-byte chunks per lane per row (K <= 1024 kChunks); kCols: columns per wave.
template <int kOut, int kChunks, int kCols>
__global__ __launch_bounds__(kGvThreads) void gemv_i8_kernel(GvArgs p) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t n0 = ((int64_t)blockIdx.x * kGvWaves + wave) * kCols;
  const int chunks = p.K >> 4;
  v4i wv[kCols][kChunks];
#pragma unroll
  for (int c = 0; c < kCols; ++c) {
    const bool col_on = n0 + c < p.N;
    const int8_t* wr = p.w + (col_on ? n0 + c : 0) * (int64_t)p.K;
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const int ch = j * kWave + lane;
      wv[c][j] = (col_on && ch < chunks) ? __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wr + (int64_t)ch * 16))
                                         : v4i{0, 0, 0, 0};
    }
  }
  v4i xv[kChunks];
#pragma unroll
  for (int j = 0; j < kChunks; ++j) {
    const int ch = j * kWave + lane;
    xv[j] = ch < chunks ? *reinterpret_cast<const v4i*>(p.xq + (int64_t)ch * 16) : v4i{0, 0, 0, 0};
  }
  const float s = p.xs[0];
#pragma unroll
  for (int c = 0; c < kCols; ++c) {
    int acc = 0;
#pragma unroll
    for (int j = 0; j < kChunks; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_sdot4(xv[j][e], wv[c][j][e], acc, false);
    acc = wave_sum_i32(acc);
    const int64_t n = n0 + c;
    if (lane == 0 && n < p.N) {
      typedef typename OutT<kOut>::T T;
      const float wsn = p.ws[p.ws_per_channel ? n : 0];
      const float b = p.bias ? OutT<kOut>::load(reinterpret_cast<const T*>(p.bias) + n) : -0.0f;
      const float y = OutT<kOut>::round((float)acc * (s * wsn));
      store_out<kOut>(reinterpret_cast<T*>(p.out) + n, y + b);
    }
  }
}

template <int kOut, int kChunks>
int launch_gemv_c(const GvArgs& a, hipStream_t st) {
  // Columns per wave: many small waves rather than ~16 KB of weights in flight per wave (measured
  // on [N, K] weights cycled from HBM, 16-byte nontemporal loads: 21504 x 5376 19.3 -> 19.1 us,
  // 10240 x 8192 15.1 -> 14.6, 16384 x 4096 12.8 -> 12.0, 6144 x 2048 5.5 -> 4.6-5.0,
  // 8192 x 1024 4.6 -> 4.0-4.1 against 2, 2, 4, 8 and 8 columns a wave).
  constexpr int kCols = kChunks <= 4 ? 2 : 1;
  const int64_t per_block = (int64_t)kGvWaves * kCols;
  const int64_t blocks = (a.N + per_block - 1) / per_block;
  if (blocks > 0x7FFFFFFF) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "N too large");
  gemv_i8_kernel<kOut, kChunks, kCols><<<(unsigned)blocks, kGvThreads, 0, st>>>(a);
  return mxq_check_launch("gemv_i8_kernel");
}

template <int kOut>
int launch_gemv_o(const GvArgs& a, hipStream_t st) {
  const int per_lane = (a.K + 1023) / 1024;
  if (per_lane <= 1) return launch_gemv_c<kOut, 1>(a, st);
  if (per_lane <= 2) return launch_gemv_c<kOut, 2>(a, st);
  if (per_lane <= 3) return launch_gemv_c<kOut, 3>(a, st);
  if (per_lane <= 4) return launch_gemv_c<kOut, 4>(a, st);
  if (per_lane <= 6) return launch_gemv_c<kOut, 6>(a, st);
  if (per_lane <= 8) return launch_gemv_c<kOut, 8>(a, st);
  if (per_lane <= 12) return launch_gemv_c<kOut, 12>(a, st);
  return launch_gemv_c<kOut, 16>(a, st);
}

int launch_gemv(const GvArgs& a, int out_dtype, hipStream_t st) {
  switch (out_dtype) {
    case MXQ_DTYPE_F32: return launch_gemv_o<0>(a, st);
    case MXQ_DTYPE_F16: return launch_gemv_o<1>(a, st);
    case MXQ_DTYPE_BF16: return launch_gemv_o<2>(a, st);
    default: return mxq_set_error(MXQ_ERR_UNSUPPORTED, "output dtype code %d", out_dtype);
  }
}

int check_gemv(const void* x, const int8_t* w, const float* ws, int64_t ws_numel, void* out, int64_t N,
               int64_t K) {
  if (N < 0 || K < 0) return mxq_set_error(MXQ_ERR_INVALID, "negative shape");
  if (N == 0) return MXQ_OK;
  if (!x || !w || !ws || !out) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  if (ws_numel != 1 && ws_numel != N)
    return mxq_set_error(MXQ_ERR_INVALID, "weight scale must have 1 or N=%lld entries, got %lld", (long long)N,
                         (long long)ws_numel);
  if (K == 0 || K % 16 || K > kGvMaxK)
    return mxq_set_error(MXQ_ERR_UNSUPPORTED, "M = 1 path needs K a multiple of 16 in [16, %d], got %lld", kGvMaxK,
                         (long long)K);
  if ((uintptr_t)x % 16 || (uintptr_t)w % 16) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "x and w must be 16-byte aligned");
  return MXQ_OK;
}

}  // namespace
}  // namespace mxq

using namespace mxq;

extern "C" int mxq_int8_linear_m1(const void* x_bf16, const int8_t* w, const float* ws, int64_t ws_numel,
                                  const void* bias, void* out, int64_t N, int64_t K, int64_t group_size,
                                  int input_act, int out_dtype, int8_t* xq, float* xs, void* stream) {
  int rc = check_gemv(x_bf16, w, ws, ws_numel, out, N, K);
  if (rc || N == 0) return rc;
  if (!xq || !xs) return mxq_set_error(MXQ_ERR_INVALID, "the quantized-row workspace (xq, xs) is required");
  if ((uintptr_t)xq % 16) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "xq must be 16-byte aligned");
  rc = mxq_quantize_int8_rowwise_convrot(x_bf16, MXQ_DTYPE_BF16, xq, xs, 1, K, group_size, input_act, stream);
  if (rc) return rc;
  GvArgs a{};
  a.xq = xq; a.xs = xs; a.w = w; a.ws = ws; a.bias = bias; a.out = out;
  a.N = N; a.K = (int)K; a.ws_per_channel = ws_numel == N && N != 1;
  return launch_gemv(a, out_dtype, (hipStream_t)stream);
}

extern "C" int mxq_int8_gemv_dequant(const int8_t* xq, const float* xs, const int8_t* w, const float* ws,
                                     int64_t ws_numel, const void* bias, void* out, int64_t N, int64_t K,
                                     int out_dtype, void* stream) {
  int rc = check_gemv(xq, w, ws, ws_numel, out, N, K);
  if (rc || N == 0) return rc;
  if (!xs) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  GvArgs a{};
  a.xq = xq; a.xs = xs; a.w = w; a.ws = ws; a.bias = bias; a.out = out;
  a.N = N; a.K = (int)K; a.ws_per_channel = ws_numel == N && N != 1;
  return launch_gemv(a, out_dtype, (hipStream_t)stream);
}
