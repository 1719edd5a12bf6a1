// W4A8 on gfx950: packed int4 weights with int8 activations.
//
// Two weight formats:
//  (1) The reference's grouped format (backends/turbo/vendor/comfy_kitchen/backends/eager/
//      w4a8_int8.py:344-363): codes c are decoded to the int8 grid
//      w8 = clamp(rne(v * s_rel[n, k/G]), -127, 127), v = codebook[c] or c - 8, then an ordinary
//      int8 GEMM runs with the per-channel scale. Decode is a streaming kernel into a
//      caller-provided workspace, chunk by chunk (as w4a8_gemm.cu:133-164 does).
//  (2) Group-scaled int4 (one fp16 scale per K-group of >= 128 and output channel): the GEMM
//      unpacks nibbles in registers and applies the group scale to each group's exact int32
//      partial sum inside the K loop:
//        acc = fma(fp32(P_g), fp32(scale[g, n]), acc) for g = 0, 1, ...;  y = out(acc * xs[m]).
//
// Kernel (2) layout. A workgroup of 4 wave64s (2 x 2) owns a BM x BN tile; each wave a WM x WN
// sub-tile of v_mfma_i32_32x32x32_i8 blocks. Per 128-wide K stage:
//  * A (activations) is staged through LDS, double-buffered, with a conflict-free XOR
//    swizzle of its 16-byte chunks (w4_swz);
//  * B (weights) never touches LDS: lane (column lane%32, half h = lane/32) loads the 32 packed
//    bytes that hold k in [k0 + 64h, k0 + 64h + 64) of its column and unpacks them in registers.
//    K-step s of the stage then consumes k in [k0 + 64h + 16s, +16) on both operands (the sum
//    over k is order-free, A fragments are read with the same mapping).
//  * Nibble c is placed in the high half of an int8 as (c ^ 8) << 4 = 16 (c - 8), so the MFMA
//    produces 16 P_g exactly; fp32(16 P) = 16 fp32(P) and fma(16P, s, 16acc) = 16 fma(P, s, acc)
//    exactly, and the final multiply uses xs / 16, so the result is bit-identical to the
//    unscaled recipe while the unpack costs 6 ALU ops per 8 weights.

#include <algorithm>
#include <mutex>

#include "w4a8_common.h"

namespace mxq {

// ---------------------------------------------------------------------------------------
// (1) grouped decode to int8
// ---------------------------------------------------------------------------------------

MXQ_DEVICE float e4m3fn_to_f32(uint32_t b) {
  const uint32_t s = b & 0x80u, e = (b >> 3) & 0xFu, m = b & 7u;
  float v;
  if ((b & 0x7Fu) == 0x7Fu) return __uint_as_float(0x7FC00000u);
  if (e == 0)
    v = (float)m * 0.001953125f;  // m / 8 * 2^-6
  else
    v = __uint_as_float(((e + 120u) << 23) | (m << 20));  // (1 + m/8) 2^(e-7)
  return s ? -v : v;
}

template <bool kE4M3>
__global__ __launch_bounds__(256) void decode_int4_grouped_kernel(
    const uint8_t* __restrict__ qdata, const void* __restrict__ s_rel,
    const float* __restrict__ codebook, int8_t* __restrict__ out, int64_t total_vec,
    int64_t k_half, int64_t groups, int group_size, int gshift) {
  __shared__ float s_cb[16];
  if (threadIdx.x < 16) s_cb[threadIdx.x] = codebook ? codebook[threadIdx.x] : (float)threadIdx.x - 8.0f;
  __syncthreads();
  for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < total_vec;
       v += (int64_t)gridDim.x * blockDim.x) {
    // 8 packed bytes -> 16 weights of one row (K % 16 == 0 keeps them in one row).
    // The vector's 16 weights lie in 16 / G groups (G = 4, 8) or in one (G a multiple of 16):
    // their scales are read once per vector, and weight i takes scale i >> gshift (gshift =
    // log2 G, or 4 for G >= 16), so no division runs per weight.
    const int64_t byte0 = v * 8;
    const int64_t n = byte0 / k_half;
    const int k0 = (int)((byte0 - n * k_half) * 2);
    const int64_t g0 = n * groups + k0 / group_size;
    const v2u w = *reinterpret_cast<const v2u*>(qdata + byte0);
    const int ng = group_size >= 16 ? 1 : 16 / group_size;
    float sv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t gi = g0 + (j < ng ? j : 0);
      sv[j] = kE4M3 ? e4m3fn_to_f32(reinterpret_cast<const uint8_t*>(s_rel)[gi])
                    : reinterpret_cast<const float*>(s_rel)[gi];
    }
    uint32_t o[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t byte = (w[i >> 3] >> (8 * ((i >> 1) & 3))) & 0xFFu;
      const uint32_t c = (i & 1) ? (byte >> 4) : (byte & 0xFu);
      const int j = i >> gshift;
      const float s = j == 0 ? sv[0] : (j == 1 ? sv[1] : (j == 2 ? sv[2] : sv[3]));
      float r = __builtin_rintf(s_cb[c] * s);
      r = fminf(fmaxf(r, -127.0f), 127.0f);
      const int q = (r != r) ? 0 : (int)r;
      o[i >> 2] |= (uint32_t)(q & 0xFF) << (8 * (i & 3));
    }
    *reinterpret_cast<v4u*>(out + n * (k_half * 2) + k0) = v4u{o[0], o[1], o[2], o[3]};
  }
}

static int decode_launch(const int8_t* qdata, const void* s_rel, int s_rel_dtype,
                         const float* codebook, int8_t* out, int64_t N, int64_t K,
                         int64_t group_size, hipStream_t st) {
  const int64_t k_half = K / 2, total_vec = N * k_half / 8, groups = K / group_size;
  int64_t blocks = (total_vec + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (total_vec == 0) return MXQ_OK;
  const int gshift = group_size == 4 ? 2 : (group_size == 8 ? 3 : 4);  // G = 4, 8 or 16 * j
  if (s_rel_dtype == MXQ_DTYPE_E4M3)
    decode_int4_grouped_kernel<true><<<(unsigned)blocks, 256, 0, st>>>(
        (const uint8_t*)qdata, s_rel, codebook, out, total_vec, k_half, groups, (int)group_size, gshift);
  else
    decode_int4_grouped_kernel<false><<<(unsigned)blocks, 256, 0, st>>>(
        (const uint8_t*)qdata, s_rel, codebook, out, total_vec, k_half, groups, (int)group_size, gshift);
  return mxq_check_launch("decode_int4_grouped_kernel");
}

static int check_decode_args(const int8_t* qdata, const void* s_rel, int s_rel_dtype,
                             int64_t N, int64_t K, int64_t G) {
  if (N < 0 || K < 0) return mxq_set_error(MXQ_ERR_INVALID, "negative shape");
  if (G < 4 || (16 % G != 0 && G % 16 != 0) || K % 16 != 0 || K % G != 0)
    return mxq_set_error(MXQ_ERR_INVALID,
                         "K=%lld must be divisible by 16 and group_size=%lld; group_size must be "
                         ">=4 and divide 16 or be a multiple of 16",
                         (long long)K, (long long)G);
  if (s_rel_dtype != MXQ_DTYPE_F32 && s_rel_dtype != MXQ_DTYPE_E4M3)
    return mxq_set_error(MXQ_ERR_UNSUPPORTED, "s_rel dtype code %d", s_rel_dtype);
  if (N > 0 && K > 0 && (!qdata || !s_rel)) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  if ((uintptr_t)qdata % 8) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "qdata must be 8-byte aligned");
  if (K > (int64_t{1} << 30)) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "K=%lld too large", (long long)K);
  return MXQ_OK;
}

// ---------------------------------------------------------------------------------------
// (2) group-scaled int4 GEMM
// ---------------------------------------------------------------------------------------

MXQ_DEVICE int w4_swz(int r, int c) { return r * kW4BK + ((c ^ (r & 7) ^ ((r >> 3) & 1)) << 4); }

template <int BM, int BN, int WM, int WN, int kOut>
__global__ __launch_bounds__(256, 1) void w4a8_grouped_kernel(W4Args p) {
  constexpr int WGM = BM / WM, WGN = BN / WN;
  static_assert(WGM * WGN == 4, "four waves per workgroup");
  constexpr int FI = WM / 32, FJ = WN / 32;
  constexpr int kStage = BM * kW4BK;
  constexpr int kArows = BM / 32;  // A rows per thread per stage (256 threads, 8 per row)
  __shared__ __attribute__((aligned(16))) char lds[2 * kStage];

  // XCD-aware, grouped tile order (see the W8A8 GEMM).
  int tm, tn;
  {
    const int num = p.tiles_m * p.tiles_n, per = num / 8, bid = blockIdx.x;
    int t = bid < per * 8 ? (bid % 8) * per + bid / 8 : bid;
    const int group = 8 * p.tiles_n, g = t / group, first = g * 8;
    const int gm = min(p.tiles_m - first, 8), in = t % group;
    tm = first + in % gm;
    tn = in / gm;
  }
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wm = wave / WGN, wn = wave % WGN;
  const int lr = lane & 31, lh = lane >> 5;
  const int64_t khalf = p.K / 2;

  v16i acc[FI][FJ];
  float facc[FI][FJ][16];
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j) {
      acc[i][j] = v16i{};
#pragma unroll
      for (int r = 0; r < 16; ++r) facc[i][j][r] = 0.0f;
    }

  // Columns this lane feeds as B operand (clamped; out-of-range columns are never stored).
  const uint8_t* wrow[FJ];
  int64_t colv[FJ];
#pragma unroll
  for (int j = 0; j < FJ; ++j) {
    colv[j] = n0 + wn * WN + j * 32 + lr;
    wrow[j] = p.w + min(colv[j], p.N - 1) * khalf + lh * 32;
  }

  auto load_a = [&](v4u* ra, int64_t k0) {
    const int c = threadIdx.x & 7;
#pragma unroll
    for (int i = 0; i < kArows; ++i) {
      const int r = (threadIdx.x >> 3) + 32 * i;
      const int64_t am = min(m0 + r, p.M - 1);
      ra[i] = *reinterpret_cast<const v4u*>(p.a + am * p.K + k0 + c * 16);
    }
  };
  auto store_a = [&](const v4u* ra, char* buf) {
    const int c = threadIdx.x & 7;
#pragma unroll
    for (int i = 0; i < kArows; ++i) {
      const int r = (threadIdx.x >> 3) + 32 * i;
      *reinterpret_cast<v4u*>(buf + w4_swz(r, c)) = ra[i];
    }
  };
  auto load_b = [&](v4u (*rb)[2], int64_t k0) {
#pragma unroll
    for (int j = 0; j < FJ; ++j) {
      const v4u* src = reinterpret_cast<const v4u*>(wrow[j] + k0 / 2);
      rb[j][0] = src[0];
      rb[j][1] = src[1];
    }
  };

  const int ktiles = (int)(p.K / kW4BK);
  v4u ra[kArows];
  v4u rb[FJ][2], rb_next[FJ][2];
  load_a(ra, 0);
  load_b(rb, 0);
  store_a(ra, lds);
  __syncthreads();

  for (int kt = 0; kt < ktiles; ++kt) {
    const char* cur = lds + (kt & 1) * kStage;
    const bool more = kt + 1 < ktiles;
    if (more) {
      load_a(ra, (int64_t)(kt + 1) * kW4BK);
      load_b(rb_next, (int64_t)(kt + 1) * kW4BK);
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      v4i fb[FJ];
#pragma unroll
      for (int j = 0; j < FJ; ++j) {
        const uint32_t w0 = rb[j][ks >> 1][(ks & 1) * 2], w1 = rb[j][ks >> 1][(ks & 1) * 2 + 1];
        uint32_t o0, o1, o2, o3;
        unpack8(w0, o0, o1);
        unpack8(w1, o2, o3);
        fb[j] = v4i{(int)o0, (int)o1, (int)o2, (int)o3};
      }
      const int c = lh * 4 + ks;
#pragma unroll
      for (int i = 0; i < FI; ++i) {
        const v4i fa = *reinterpret_cast<const v4i*>(cur + w4_swz(wm * WM + i * 32 + lr, c));
#pragma unroll
        for (int j = 0; j < FJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa, fb[j], acc[i][j], 0, 0, 0);
      }
    }
    // End of a group: fold 16 P_g into the fp32 accumulators with the group's scales.
    if ((kt + 1) % p.group_tiles == 0) {
      const int64_t g = kt / p.group_tiles;
#pragma unroll
      for (int j = 0; j < FJ; ++j) {
        const float s = f16_to_f32(p.gs[g * p.N + min(colv[j], p.N - 1)]);
#pragma unroll
        for (int i = 0; i < FI; ++i) {
#pragma unroll
          for (int r = 0; r < 16; ++r) facc[i][j][r] = fmaf((float)acc[i][j][r], s, facc[i][j][r]);
          acc[i][j] = v16i{};
        }
      }
    }
    if (more) {
      store_a(ra, lds + ((kt + 1) & 1) * kStage);
#pragma unroll
      for (int j = 0; j < FJ; ++j) {
        rb[j][0] = rb_next[j][0];
        rb[j][1] = rb_next[j][1];
      }
    }
    __syncthreads();
  }

  // Epilogue: y = out(acc * (xs / 16)); y = out(y + bias).
  typedef typename OutT<kOut>::T OT;
  OT* D = reinterpret_cast<OT*>(p.d);
  const OT* bias = reinterpret_cast<const OT*>(p.bias);
#pragma unroll
  for (int j = 0; j < FJ; ++j) {
    const int64_t col = colv[j];
    const float bv = bias ? OutT<kOut>::load(bias + min(col, p.N - 1)) : 0.0f;
#pragma unroll
    for (int i = 0; i < FI; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm * WM + i * 32 + (r >> 2) * 8 + lh * 4 + (r & 3);
        const float xs16 = p.xs[min(row, p.M - 1)] * 0.0625f;
        float y = OutT<kOut>::round(facc[i][j][r] * xs16);
        if (bias) y = OutT<kOut>::round(y + bv);
        if (row < p.M && col < p.N) store_out<kOut>(D + row * p.ldd + col, y);
      }
    }
  }
}

template <int BM, int BN, int WM, int WN>
static int launch_w4(W4Args p, int out_dtype, hipStream_t st) {
  p.tiles_m = (int)((p.M + BM - 1) / BM);
  p.tiles_n = (int)((p.N + BN - 1) / BN);
  const unsigned grid = (unsigned)(p.tiles_m * p.tiles_n);
  switch (out_dtype) {
    case MXQ_DTYPE_F32: w4a8_grouped_kernel<BM, BN, WM, WN, 0><<<grid, 256, 0, st>>>(p); break;
    case MXQ_DTYPE_F16: w4a8_grouped_kernel<BM, BN, WM, WN, 1><<<grid, 256, 0, st>>>(p); break;
    case MXQ_DTYPE_BF16: w4a8_grouped_kernel<BM, BN, WM, WN, 2><<<grid, 256, 0, st>>>(p); break;
    default: return mxq_set_error(MXQ_ERR_UNSUPPORTED, "output dtype code %d", out_dtype);
  }
  return mxq_check_launch("w4a8_grouped_kernel");
}

}  // namespace mxq

using namespace mxq;

extern "C" int mxq_dequant_int4_grouped_to_int8(const int8_t* qdata, const void* s_rel,
                                                int s_rel_dtype, const float* codebook,
                                                int8_t* out, int64_t N, int64_t K,
                                                int64_t group_size, void* stream) {
  int rc = check_decode_args(qdata, s_rel, s_rel_dtype, N, K, group_size);
  if (rc) return rc;
  if (N == 0 || K == 0) return MXQ_OK;
  if (!out) return mxq_set_error(MXQ_ERR_INVALID, "null output");
  if ((uintptr_t)out % 16) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "output must be 16-byte aligned");
  return decode_launch(qdata, s_rel, s_rel_dtype, codebook, out, N, K, group_size, (hipStream_t)stream);
}

// Decode-then-GEMM over column chunks of chunk_cols weights rows, the decoded chunk in
// `workspace` ([chunk_cols, K] int8), each chunk's GEMM with the tile-queue workspace `queue`
// (NULL: static tile order). Arguments are validated by the callers.
static int codebook_gemm_chunks(const int8_t* xq, const int8_t* qdata, const void* s_rel, int s_rel_dtype,
                                const float* codebook, const float* s_channel, const float* xs,
                                const void* bias, int8_t* workspace, void* out, int64_t M, int64_t N,
                                int64_t K, int64_t group_size, int64_t chunk_cols, int out_dtype,
                                void* queue, int64_t queue_bytes, void* stream) {
  const int osz = out_dtype == MXQ_DTYPE_F32 ? 4 : 2;
  const int64_t groups = K / group_size;
  const int sbytes = s_rel_dtype == MXQ_DTYPE_E4M3 ? 1 : 4;
  hipStream_t st = (hipStream_t)stream;
  for (int64_t n0 = 0; n0 < N; n0 += chunk_cols) {
    const int64_t cols = chunk_cols < N - n0 ? chunk_cols : N - n0;
    int rc = decode_launch(qdata + n0 * (K / 2), (const char*)s_rel + n0 * groups * sbytes,
                           s_rel_dtype, codebook, workspace, cols, K, group_size, st);
    if (rc) return rc;
    const void* bias_chunk = bias ? (const char*)bias + n0 * osz : nullptr;
    rc = mxq_int8_gemm_dequant(xq, workspace, xs, s_channel + n0, cols, bias_chunk,
                               (char*)out + n0 * osz, M, cols, K, N, out_dtype, queue, queue_bytes, stream);
    if (rc) return rc;
  }
  return MXQ_OK;
}

static int check_codebook_gemm(const int8_t* qdata, const void* s_rel, int s_rel_dtype,
                               const float* s_channel, const float* xs, const void* out, int64_t M,
                               int64_t N, int64_t K, int64_t group_size, int64_t chunk_cols) {
  int rc = check_decode_args(qdata, s_rel, s_rel_dtype, N, K, group_size);
  if (rc) return rc;
  if (M < 0) return mxq_set_error(MXQ_ERR_INVALID, "negative M");
  if (M == 0 || N == 0) return MXQ_OK;
  if (chunk_cols <= 0) return mxq_set_error(MXQ_ERR_INVALID, "chunk_cols must be positive");
  if (!out || !s_channel || !xs) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  return MXQ_OK;
}

extern "C" int mxq_w4a8_codebook_gemm(const int8_t* xq, const int8_t* qdata, const void* s_rel,
                                      int s_rel_dtype, const float* codebook,
                                      const float* s_channel, const float* xs, const void* bias,
                                      int8_t* workspace, void* out, int64_t M, int64_t N,
                                      int64_t K, int64_t group_size, int64_t chunk_cols,
                                      int out_dtype, void* gemm_workspace, int64_t gemm_workspace_bytes,
                                      void* stream) {
  int rc = check_codebook_gemm(qdata, s_rel, s_rel_dtype, s_channel, xs, out, M, N, K, group_size, chunk_cols);
  if (rc || M == 0 || N == 0) return rc;
  if (!workspace) return mxq_set_error(MXQ_ERR_INVALID, "null workspace");
  return codebook_gemm_chunks(xq, qdata, s_rel, s_rel_dtype, codebook, s_channel, xs, bias, workspace, out, M, N,
                              K, group_size, chunk_cols, out_dtype, gemm_workspace, gemm_workspace_bytes, stream);
}

// ---- allocation-free variant ----------------------------------------------------------
// The decode workspace of mxq_w4a8_codebook_gemm_noalloc is this file-scope array: each GPU the
// library runs on holds its own copy (kNoAllocScratchBytes) until the process ends. Host code
// never passes `scratch` itself to a kernel (in host code the name is a host-side stand-in, not a
// device address): the device address is looked up once per device with hipGetSymbolAddress and
// kept in g_scratch_ptr. Every call on one GPU reuses that GPU's array; the decode overwrites
// every byte a GEMM reads, so nothing needs clearing between calls. Every call first makes its
// stream wait for the previous call on the same GPU (an event recorded after every call, created
// with the address lookup), so calls from two streams do not overlap. Under graph capture neither the wait nor the record is made (the
// graph's own edges order its calls), so a replayed graph that runs beside another call on the
// same GPU races with it on the array. The chunk GEMMs' tile-queue counters are a second, small
// array of the same kind (zero when the library loads; every GEMM leaves them zero).
constexpr int64_t kNoAllocScratchBytes = int64_t(32) << 20;
static __device__ __attribute__((aligned(256))) int8_t scratch[kNoAllocScratchBytes];
static __device__ __attribute__((aligned(256))) uint32_t queue_scratch[MXQ_GEMM_WORKSPACE_BYTES / 4];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
int8_t* g_scratch_ptr[kMaxScratchDevices] = {};
void* g_queue_ptr[kMaxScratchDevices] = {};
hipEvent_t g_last_call[kMaxScratchDevices] = {};  // recorded after each call on the device

// Device addresses of the current device's scratch and queue arrays and its call-order event
// (looked up and created on the first call per device). The caller holds g_scratch_mutex.
int current_device_scratch(int* device, int8_t** ptr, void** queue) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return mxq_set_error(MXQ_ERR_HIP, "hipGetDevice failed: %s", hipGetErrorString(err));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return mxq_set_error(MXQ_ERR_UNSUPPORTED, "device ordinal %d outside the %d the library tracks", dev,
                         kMaxScratchDevices);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || p == nullptr)
      return mxq_set_error(MXQ_ERR_HIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                           hipGetErrorString(err));
    void* qp = nullptr;
    err = hipGetSymbolAddress(&qp, HIP_SYMBOL(queue_scratch));
    if (err != hipSuccess || qp == nullptr)
      return mxq_set_error(MXQ_ERR_HIP, "hipGetSymbolAddress(queue_scratch) failed on device %d: %s", dev,
                           hipGetErrorString(err));
    hipEvent_t ev = nullptr;
    err = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (err != hipSuccess)
      return mxq_set_error(MXQ_ERR_HIP, "hipEventCreateWithFlags failed on device %d: %s", dev, hipGetErrorString(err));
    g_scratch_ptr[dev] = static_cast<int8_t*>(p);
    g_queue_ptr[dev] = qp;
    g_last_call[dev] = ev;
  }
  *device = dev;
  *ptr = g_scratch_ptr[dev];
  *queue = g_queue_ptr[dev];
  return MXQ_OK;
}
}  // namespace

extern "C" int mxq_w4a8_codebook_gemm_noalloc(const int8_t* xq, const int8_t* qdata, const void* s_rel,
                                              int s_rel_dtype, const float* codebook,
                                              const float* s_channel, const float* xs, const void* bias,
                                              void* out, int64_t M, int64_t N, int64_t K, int64_t group_size,
                                              int64_t chunk_cols, int out_dtype, void* stream) {
  int rc = check_codebook_gemm(qdata, s_rel, s_rel_dtype, s_channel, xs, out, M, N, K, group_size, chunk_cols);
  if (rc || M == 0 || N == 0) return rc;
  const int64_t cols = chunk_cols < N ? chunk_cols : N;
  if (cols > kNoAllocScratchBytes / K)
    return mxq_set_error(MXQ_ERR_INVALID,
                         "decode chunk of %lld x %lld int8 exceeds the %lld-byte static workspace; use at most "
                         "%lld columns per chunk",
                         (long long)cols, (long long)K, (long long)kNoAllocScratchBytes,
                         (long long)(kNoAllocScratchBytes / K));
  int8_t* ws = nullptr;
  void* queue = nullptr;
  int dev = -1;
  hipStream_t st = (hipStream_t)stream;
  // Host threads take turns: the order wait, the launches and the order record happen under the
  // lock, so no other call's launches come between them.
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  rc = current_device_scratch(&dev, &ws, &queue);
  if (rc) return rc;
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  hipError_t err = hipStreamIsCapturing(st, &capture);
  if (err != hipSuccess) return mxq_set_error(MXQ_ERR_HIP, "hipStreamIsCapturing failed: %s", hipGetErrorString(err));
  const bool order = capture == hipStreamCaptureStatusNone;
  if (order) {  // (also on the same stream, where it orders nothing new: a stream handle can be reused)
    err = hipStreamWaitEvent(st, g_last_call[dev], 0);
    if (err != hipSuccess) return mxq_set_error(MXQ_ERR_HIP, "hipStreamWaitEvent failed: %s", hipGetErrorString(err));
  }
  rc = codebook_gemm_chunks(xq, qdata, s_rel, s_rel_dtype, codebook, s_channel, xs, bias, ws, out, M, N, K,
                            group_size, chunk_cols, out_dtype, queue, MXQ_GEMM_WORKSPACE_BYTES, stream);
  if (rc) return rc;
  if (order) {
    err = hipEventRecord(g_last_call[dev], st);
    if (err != hipSuccess) return mxq_set_error(MXQ_ERR_HIP, "hipEventRecord failed: %s", hipGetErrorString(err));
  }
  return MXQ_OK;
}

static int check_grouped(const int8_t* a, const float* xs, const int8_t* qdata, const uint16_t* group_scale,
                         void* d, int64_t M, int64_t N, int64_t K, int64_t group_size, int64_t ldd) {
  if (M < 0 || N < 0 || K < 0) return mxq_set_error(MXQ_ERR_INVALID, "negative shape");
  if (M == 0 || N == 0) return MXQ_OK;
  if (!a || !xs || !qdata || !group_scale || !d) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  if (group_size <= 0 || group_size % kW4BK != 0 || K % group_size != 0 || K == 0)
    return mxq_set_error(MXQ_ERR_UNSUPPORTED,
                         "grouped W4A8 needs group_size a multiple of 128 dividing K (K=%lld, G=%lld)",
                         (long long)K, (long long)group_size);
  if (ldd < N) return mxq_set_error(MXQ_ERR_INVALID, "output stride < N");
  if (K > 131072) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "K too large");
  if ((uintptr_t)a % 16 || (uintptr_t)qdata % 16)
    return mxq_set_error(MXQ_ERR_UNSUPPORTED, "A and packed weights must be 16-byte aligned");
  return MXQ_OK;
}

static W4Args grouped_args(const int8_t* a, const float* xs, const int8_t* qdata, const uint16_t* group_scale,
                           const void* bias, void* d, int64_t M, int64_t N, int64_t K, int64_t group_size,
                           int64_t ldd) {
  W4Args p{};
  p.a = a; p.xs = xs; p.w = (const uint8_t*)qdata; p.gs = group_scale; p.bias = bias; p.d = d;
  p.M = M; p.N = N; p.K = K; p.ldd = ldd; p.group_tiles = (int)(group_size / kW4BK);
  return p;
}

extern "C" int mxq_w4a8_gemm_grouped(const int8_t* a, const float* xs, const int8_t* qdata,
                                     const uint16_t* group_scale, const void* bias, void* d,
                                     int64_t M, int64_t N, int64_t K, int64_t group_size,
                                     int64_t ldd, int out_dtype, void* stream) {
  const int rc0 = check_grouped(a, xs, qdata, group_scale, d, M, N, K, group_size, ldd);
  if (rc0 != MXQ_OK || M == 0 || N == 0) return rc0;
  const W4Args p = grouped_args(a, xs, qdata, group_scale, bias, d, M, N, K, group_size, ldd);
  hipStream_t st = (hipStream_t)stream;
  // Group 128 (one group per K stage) with 16-byte aligned scale rows: the pipelined kernel on
  // 128 x 128 tiles, two workgroups per CU.
  if (group_size == 128 && N % 8 == 0 && (uintptr_t)group_scale % 16 == 0) {
    const int rc = launch_w4_g128(p, out_dtype, false, st);
    if (rc != MXQ_ERR_UNSUPPORTED) return rc;  // else: operands too large for 32-bit offsets
  }
  // Other group sizes: 256 x 128 tiles (waves 128 x 64) for large M, 128 x 64 otherwise.
  if (M >= 2048) return launch_w4<256, 128, 128, 64>(p, out_dtype, st);
  return launch_w4<128, 64, 64, 32>(p, out_dtype, st);
}

extern "C" int mxq_w4a8_gemm_grouped_prepared(const int8_t* a, const float* xs, const int8_t* qdata,
                                              const uint16_t* group_scale, const void* bias, void* d,
                                              int64_t M, int64_t N, int64_t K, int64_t group_size,
                                              int64_t ldd, int out_dtype, void* stream) {
  const int rc0 = check_grouped(a, xs, qdata, group_scale, d, M, N, K, group_size, ldd);
  if (rc0 != MXQ_OK || M == 0 || N == 0) return rc0;
  if (group_size != 128 || N % 8 != 0 || (uintptr_t)group_scale % 16 != 0)
    return mxq_set_error(MXQ_ERR_UNSUPPORTED,
                         "prepared W4A8 weights need group 128, N %% 8 == 0 and 16-byte aligned scales "
                         "(G=%lld, N=%lld)", (long long)group_size, (long long)N);
  const W4Args p = grouped_args(a, xs, qdata, group_scale, bias, d, M, N, K, group_size, ldd);
  const int rc = launch_w4_g128(p, out_dtype, true, (hipStream_t)stream);
  if (rc == MXQ_ERR_UNSUPPORTED)
    return mxq_set_error(MXQ_ERR_UNSUPPORTED, "prepared W4A8 operands exceed 2^31 bytes (M=%lld, N=%lld, K=%lld)",
                         (long long)M, (long long)N, (long long)K);
  return rc;
}

namespace mxq {
namespace {

// One 32-bit word (8 codes of k = 8w .. 8w + 7) per thread, grid-stride; in place allowed.
__global__ __launch_bounds__(256) void w4_prepare_kernel(const uint32_t* in, uint32_t* out, int64_t words) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += stride) {
    const uint32_t w = in[i] ^ 0x88888888u;  // every code c -> c ^ 8, the 4-bit value c - 8
    uint32_t r = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      r |= (((w >> (4 * j)) & 0xFu) | (((w >> (4 * (4 + j))) & 0xFu) << 4)) << (8 * j);
    out[i] = r;
  }
}

}  // namespace
}  // namespace mxq

namespace mxq {
namespace {

// sx[m, g] = out(out(sum of xq[m, k] over group g) * out(xs[m])), one output per thread.
template <int kOut>
__global__ __launch_bounds__(256) void group_sums_kernel(const int8_t* __restrict__ xq, const float* __restrict__ xs,
                                                         void* __restrict__ out, int64_t M, int64_t K, int64_t G) {
  typedef typename OutT<kOut>::T T;
  const int64_t groups = K / G, total = M * groups;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t m = i / groups, g = i - m * groups;
    const int8_t* src = xq + m * K + g * G;
    int sum = 0;
    for (int64_t e = 0; e < G; ++e) sum += src[e];
    const float v = OutT<kOut>::round(OutT<kOut>::round((float)sum) * OutT<kOut>::round(xs[m]));
    store_out<kOut>(reinterpret_cast<T*>(out) + i, v);
  }
}

}  // namespace
}  // namespace mxq

extern "C" int mxq_int8_group_sums(const int8_t* xq, const float* xs, void* out, int64_t M, int64_t K,
                                   int64_t group_size, int out_dtype, void* stream) {
  if (M < 0 || K < 0) return mxq_set_error(MXQ_ERR_INVALID, "negative shape");
  if (group_size <= 0 || K % group_size != 0)
    return mxq_set_error(MXQ_ERR_INVALID, "group_size=%lld must divide K=%lld", (long long)group_size, (long long)K);
  const int64_t total = M * (K / group_size);
  if (total == 0) return MXQ_OK;
  if (!xq || !xs || !out) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 65536);
  hipStream_t st = (hipStream_t)stream;
  switch (out_dtype) {
    case MXQ_DTYPE_F32: mxq::group_sums_kernel<0><<<blocks, 256, 0, st>>>(xq, xs, out, M, K, group_size); break;
    case MXQ_DTYPE_F16: mxq::group_sums_kernel<1><<<blocks, 256, 0, st>>>(xq, xs, out, M, K, group_size); break;
    case MXQ_DTYPE_BF16: mxq::group_sums_kernel<2><<<blocks, 256, 0, st>>>(xq, xs, out, M, K, group_size); break;
    default: return mxq_set_error(MXQ_ERR_UNSUPPORTED, "output dtype code %d", out_dtype);
  }
  return mxq_check_launch("group_sums_kernel");
}

extern "C" int mxq_w4a8_prepare_grouped(const int8_t* qdata, int8_t* out, int64_t N, int64_t K, void* stream) {
  if (N < 0 || K < 0) return mxq_set_error(MXQ_ERR_INVALID, "negative shape");
  if (K % 8 != 0) return mxq_set_error(MXQ_ERR_INVALID, "K=%lld must be a multiple of 8", (long long)K);
  const int64_t words = N * (K / 8);
  if (words == 0) return MXQ_OK;
  if (!qdata || !out) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  if ((uintptr_t)qdata % 4 || (uintptr_t)out % 4)
    return mxq_set_error(MXQ_ERR_UNSUPPORTED, "packed weights must be 4-byte aligned");
  const int64_t blocks = std::min<int64_t>((words + 255) / 256, 8192);
  mxq::w4_prepare_kernel<<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>(
      reinterpret_cast<const uint32_t*>(qdata), reinterpret_cast<uint32_t*>(out), words);
  return mxq_check_launch("w4_prepare_kernel");
}
