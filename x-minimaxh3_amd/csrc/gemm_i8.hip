// INT8 x INT8 -> INT32 GEMM on gfx950 matrix cores, with fused epilogues.
//
// C[m, n] = sum_k A[m, k] * B[n, k]: A [M, K] activations, B [N, K] weights, both K-contiguous
// (the reference's torch._int_mm(x_8, weight.T) / CUTLASS RowMajor x ColumnMajor,
// backends/turbo/vendor/comfy_kitchen/backends/cuda/ops/cutlass_gemm_int8.cu:245-283).
//
// Main loop: a 256-thread workgroup (4 wave64s, 2 x 2) owns a 256 x 256 output tile; each wave
// owns 128 x 128 as a 4 x 4 grid of v_mfma_i32_32x32x32_i8 blocks (256 int32 accumulators per
// lane, held in AGPRs). K advances 128 bytes per stage; A and B stages (32 KB each) are
// double-buffered in LDS. Global loads for stage k+1 are issued before the MFMAs of stage k and
// written to LDS after them, so one barrier per stage suffices.
//
// LDS operand layout: a tile row is 128 bytes = eight 16-byte chunks; chunk c of row r sits at
// slot c ^ (r & 7) ^ ((r >> 3) & 1). Eight consecutive rows then hit eight distinct 16-byte slots
// of a 128-byte bank sweep and sixteen consecutive rows distinct slots of a 256-byte sweep, so
// the MFMA operand reads (ds_read_b128, one row per lane) and the stage writes are conflict-free.
//
// Epilogue: each wave converts its accumulators in place (MFMA layout) and writes them to an
// LDS copy of the output tile; the workgroup then streams that tile to HBM row by row with
// 16-byte stores (2-byte outputs: the whole tile at once; 4-byte outputs: two halves).
//   kEpiI32     raw int32 accumulators.
//   kEpiDequant y = out(fp32(acc) * (xs[m] * ws[n])); y = out(y + bias[n])
//               (backends/eager/quantization.py:1031-1054; single IEEE ops, -ffp-contract=off).
//   kEpiGelu    bf16 dequant as above, then h = gelu_tanh(y) in bf16 while streaming out, and the
//               per-row absmax of h folded into row_absmax[m] with atomics (it feeds the next
//               layer's quantizer, backends/_activations.py:40-53 + quantization.py:857-875).

#include "mxq_common.h"

namespace mxq {

constexpr int kBM = 256, kBN = 256, kBK = 128;
constexpr int kGemmThreads = 256;
constexpr int kWaveM = 128, kWaveN = 128;
constexpr int kStageA = kBM * kBK, kStageB = kBN * kBK;
constexpr int kStageBytes = kStageA + kStageB;
constexpr int kGroupM = 8;

// Epilogue LDS map: output tile rows padded by 16 bytes (rows r and r+4, written by the two
// half-waves of one store, then land in different banks).
template <int kElem> struct EpiLayout {
  static constexpr int kRows = kElem == 2 ? kBM : kBM / 2;   // rows per pass
  static constexpr int kPitch = kBN * kElem + 16;
  static constexpr int kTile = kRows * kPitch;
  static constexpr int kFactors = kTile;                     // xs[256], ws[256], bias[256] floats
  static constexpr int kBytes = kTile + 3 * 256 * 4;
};
constexpr int kLdsBytes = EpiLayout<4>::kBytes > 2 * kStageBytes
                              ? (EpiLayout<4>::kBytes > EpiLayout<2>::kBytes ? EpiLayout<4>::kBytes : EpiLayout<2>::kBytes)
                              : 2 * kStageBytes;

enum { kEpiI32 = 0, kEpiDequant = 1, kEpiGelu = 2 };

struct GemmArgs {
  const int8_t* a;
  const int8_t* b;
  const float* xs;
  const float* ws;
  const void* bias;
  void* d;
  float* row_absmax;
  int64_t M, N, K, ldd;
  int ws_per_channel;
  int vec_store;  // 16-byte row stores allowed (d and ldd 16-byte aligned)
  int tiles_m, tiles_n;
};

MXQ_DEVICE int swz(int r, int c) { return r * kBK + ((c ^ (r & 7) ^ ((r >> 3) & 1)) << 4); }

// Tile order: first spread contiguous tile ranges over the 8 XCDs (workgroup ids are dealt to
// XCDs round-robin), then walk each range in groups of kGroupM tile-rows so that the ~32 tiles
// resident on one XCD share A and B panels in that XCD's L2.
MXQ_DEVICE void tile_coords(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int num = tiles_m * tiles_n;
  const int per = num / 8;
  int t = bid;
  if (bid < per * 8) t = (bid % 8) * per + bid / 8;
  const int group = kGroupM * tiles_n;
  const int g = t / group;
  const int first_m = g * kGroupM;
  const int gm = min(tiles_m - first_m, kGroupM);
  const int in = t % group;
  tm = first_m + in % gm;
  tn = in / gm;
}

// Global -> register staging: thread t moves chunk (t % 8) of rows t / 8 + 32 i, i = 0..7.
struct Stage {
  v4u a[8];
  v4u b[8];
};

MXQ_DEVICE void load_stage(Stage& s, const int8_t* __restrict__ A, const int8_t* __restrict__ B,
                           int64_t M, int64_t N, int64_t K, int64_t m0, int64_t n0, int64_t k0) {
  const int t = threadIdx.x;
  const int c = t & 7;
  const int64_t kk = k0 + c * 16;
  const bool kin = kk < K;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = (t >> 3) + 32 * i;
    const int64_t am = min(m0 + r, M - 1);
    const int64_t bn = min(n0 + r, N - 1);
    if (kin) {
      s.a[i] = *reinterpret_cast<const v4u*>(A + am * K + kk);
      s.b[i] = *reinterpret_cast<const v4u*>(B + bn * K + kk);
    } else {
      s.a[i] = v4u{0, 0, 0, 0};
      s.b[i] = v4u{0, 0, 0, 0};
    }
  }
}

MXQ_DEVICE void store_stage(const Stage& s, char* lds) {
  const int t = threadIdx.x;
  const int c = t & 7;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = (t >> 3) + 32 * i;
    *reinterpret_cast<v4u*>(lds + swz(r, c)) = s.a[i];
    *reinterpret_cast<v4u*>(lds + kStageA + swz(r, c)) = s.b[i];
  }
}

MXQ_DEVICE void load_frags(const char* lds, int wm, int wn, int ks, v4i fa[4], v4i fb[4]) {
  const int lane = threadIdx.x & 63;
  const int c = ks * 2 + (lane >> 5);
  const int lr = lane & 31;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    fa[i] = *reinterpret_cast<const v4i*>(lds + swz(wm * kWaveM + i * 32 + lr, c));
#pragma unroll
  for (int j = 0; j < 4; ++j)
    fb[j] = *reinterpret_cast<const v4i*>(lds + kStageA + swz(wn * kWaveN + j * 32 + lr, c));
}

MXQ_DEVICE void mma_stage(const char* lds, int wm, int wn, v16i acc[4][4]) {
  v4i fa[2][4], fb[2][4];
  load_frags(lds, wm, wn, 0, fa[0], fb[0]);
#pragma unroll
  for (int ks = 0; ks < kBK / 32; ++ks) {
    if (ks + 1 < kBK / 32) load_frags(lds, wm, wn, ks + 1, fa[(ks + 1) & 1], fb[(ks + 1) & 1]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[ks & 1][i], fb[ks & 1][j], acc[i][j],
                                                          0, 0, 0);
  }
}

// Element (i, j, r) of a lane's accumulators: tile row wm*128 + i*32 + (r/4)*8 + (lane/32)*4
// + r%4, tile column wn*128 + j*32 + lane%32 (the v_mfma_i32_32x32x32_i8 layout).
MXQ_DEVICE int acc_row(int wm, int i, int r, int lh) { return wm * kWaveM + i * 32 + (r >> 2) * 8 + lh * 4 + (r & 3); }

template <int kEpi, int kOut>
MXQ_DEVICE uint32_t epi_value(int32_t acc, float xs, float ws, float bias, bool has_bias) {
  if (kEpi == kEpiI32) return (uint32_t)acc;
  float y = OutT<kOut>::round((float)acc * (xs * ws));
  if (has_bias) y = OutT<kOut>::round(y + bias);
  if (kOut == 0) return __float_as_uint(y);
  if (kOut == 1) return f32_to_f16_bits(y);
  return f32_to_bf16_bits(y);
}

template <int kEpi, int kOut>
__global__ __launch_bounds__(kGemmThreads, 1) void gemm_i8_kernel(GemmArgs p) {
  __shared__ __attribute__((aligned(16))) char lds[kLdsBytes];

  int tm, tn;
  tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * kBM, n0 = (int64_t)tn * kBN;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wm = wave >> 1, wn = wave & 1;

  v16i acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v16i{};

  const int ktiles = (int)((p.K + kBK - 1) / kBK);
  Stage st;
  load_stage(st, p.a, p.b, p.M, p.N, p.K, m0, n0, 0);
  store_stage(st, lds);
  __syncthreads();
  for (int kt = 0; kt < ktiles; ++kt) {
    char* cur = lds + (kt & 1) * kStageBytes;
    const bool more = kt + 1 < ktiles;
    if (more) load_stage(st, p.a, p.b, p.M, p.N, p.K, m0, n0, (int64_t)(kt + 1) * kBK);
    mma_stage(cur, wm, wn, acc);
    if (more) store_stage(st, lds + ((kt + 1) & 1) * kStageBytes);
    __syncthreads();
  }

  // ---- epilogue ----
  constexpr int kElem = (kOut == 0 || kEpi == kEpiI32) ? 4 : 2;
  typedef EpiLayout<kElem> L;
  const int lr = lane & 31, lh = lane >> 5;
  const int t = threadIdx.x;
  float* s_xs = reinterpret_cast<float*>(lds + L::kFactors);
  float* s_ws = s_xs + kBM;
  float* s_bias = s_ws + kBN;
  const bool has_bias = p.bias != nullptr;
  if (kEpi != kEpiI32) {
    const int64_t row = min(m0 + t, p.M - 1);
    const int64_t col = min(n0 + t, p.N - 1);
    s_xs[t] = p.xs[row];
    s_ws[t] = p.ws_per_channel ? p.ws[col] : p.ws[0];
    s_bias[t] = has_bias ? OutT<kOut>::load(reinterpret_cast<const typename OutT<kOut>::T*>(p.bias) + col) : 0.0f;
    __syncthreads();
  }

  constexpr int kPasses = kBM / L::kRows;
  constexpr int kCpr = kBN * kElem / 16;  // 16-byte chunks per tile row
  constexpr int kPerRow = 16 / kElem;     // elements per chunk
#pragma unroll
  for (int pass = 0; pass < kPasses; ++pass) {
    if (kPasses == 1 || wm == pass) {
      const int rbase = (kPasses == 1) ? 0 : pass * L::kRows;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int cl = wn * kWaveN + j * 32 + lr;
          const float wsv = s_ws[cl], bv = s_bias[cl];
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int rl = acc_row(wm, i, r, lh);
            const uint32_t v = epi_value<kEpi, kOut>(acc[i][j][r], s_xs[rl], wsv, bv, has_bias);
            char* dst = lds + (rl - rbase) * L::kPitch + cl * kElem;
            if (kElem == 4)
              *reinterpret_cast<uint32_t*>(dst) = v;
            else
              *reinterpret_cast<uint16_t*>(dst) = (uint16_t)v;
          }
        }
    }
    __syncthreads();

    // Stream the LDS tile out: each 16-byte chunk of a row to HBM; a half-wave covers one row.
    constexpr int kIters = L::kRows * kCpr / kGemmThreads;
#pragma unroll 4
    for (int it = 0; it < kIters; ++it) {
      const int idx = it * kGemmThreads + t;
      const int rl = idx / kCpr, c = idx % kCpr;
      v4u v = *reinterpret_cast<const v4u*>(lds + rl * L::kPitch + c * 16);
      const int64_t row = m0 + pass * L::kRows + rl;
      const int64_t col = n0 + c * kPerRow;
      float m = 0.0f;
      if (kEpi == kEpiGelu) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t lo = gelu_bf16(v[w] & 0xFFFFu), hi = gelu_bf16(v[w] >> 16);
          v[w] = lo | (hi << 16);
          if (col + 2 * w < p.N) m = fmaxf(m, fabsf(bf16_to_f32(lo)));
          if (col + 2 * w + 1 < p.N) m = fmaxf(m, fabsf(bf16_to_f32(hi)));
        }
      }
      if (row < p.M) {
        char* out = reinterpret_cast<char*>(p.d) + (row * p.ldd + col) * kElem;
        if (p.vec_store && col + kPerRow <= p.N) {
          *reinterpret_cast<v4u*>(out) = v;
        } else {
#pragma unroll
          for (int e = 0; e < kPerRow; ++e) {
            if (col + e < p.N) {
              if (kElem == 4)
                reinterpret_cast<uint32_t*>(out)[e] = v[e];
              else
                reinterpret_cast<uint16_t*>(out)[e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
            }
          }
        }
      }
      if (kEpi == kEpiGelu) {
        // kCpr == 32: lanes 0-31 and 32-63 of a wave each hold one full tile row.
        m = halfwave_max(m);
        if ((lane & 31) == 0 && row < p.M) atomic_max_nonneg(p.row_absmax + row, m);
      }
    }
    if (kPasses > 1) __syncthreads();
  }
}

template <int kEpi, int kOut>
static int launch_gemm(const GemmArgs& args0, hipStream_t stream) {
  GemmArgs args = args0;
  args.tiles_m = (int)((args.M + kBM - 1) / kBM);
  args.tiles_n = (int)((args.N + kBN - 1) / kBN);
  const int elem = (kOut == 0 || kEpi == kEpiI32) ? 4 : 2;
  args.vec_store = ((uintptr_t)args.d % 16 == 0) && ((args.ldd * elem) % 16 == 0);
  const int64_t tiles = (int64_t)args.tiles_m * args.tiles_n;
  if (tiles > INT32_MAX) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "too many tiles");
  gemm_i8_kernel<kEpi, kOut><<<(unsigned)tiles, kGemmThreads, 0, stream>>>(args);
  return mxq_check_launch("gemm_i8_kernel");
}

static int check_gemm_shape(const int8_t* a, const int8_t* b, const void* d, int64_t M, int64_t N,
                            int64_t K, int64_t ldd) {
  if (M < 0 || N < 0 || K < 0) return mxq_set_error(MXQ_ERR_INVALID, "negative GEMM shape");
  if (M > 0 && N > 0 && (!a || !b || !d)) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  if (ldd < N) return mxq_set_error(MXQ_ERR_INVALID, "output stride %lld < N %lld", (long long)ldd, (long long)N);
  if (M > 0 && N > 0 && K == 0) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "K == 0");
  if (K % 16 != 0) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "K=%lld must be a multiple of 16", (long long)K);
  if (K > 131056) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "K=%lld exceeds the int32 accumulator bound", (long long)K);
  if ((uintptr_t)a % 16 || (uintptr_t)b % 16) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "A and B must be 16-byte aligned");
  return MXQ_OK;
}

}  // namespace mxq

using namespace mxq;

extern "C" int mxq_int8_gemm_i32(const int8_t* a, const int8_t* b, int32_t* c, int64_t M,
                                 int64_t N, int64_t K, int64_t ldc, void* stream) {
  int rc = check_gemm_shape(a, b, c, M, N, K, ldc);
  if (rc) return rc;
  if (M == 0 || N == 0) return MXQ_OK;
  GemmArgs g{};
  g.a = a; g.b = b; g.d = c; g.M = M; g.N = N; g.K = K; g.ldd = ldc;
  return launch_gemm<kEpiI32, 0>(g, (hipStream_t)stream);
}

extern "C" int mxq_int8_gemm_dequant(const int8_t* a, const int8_t* b, const float* xs,
                                     const float* ws, int64_t ws_numel, const void* bias, void* d,
                                     int64_t M, int64_t N, int64_t K, int64_t ldd, int out_dtype,
                                     void* stream) {
  int rc = check_gemm_shape(a, b, d, M, N, K, ldd);
  if (rc) return rc;
  if (M == 0 || N == 0) return MXQ_OK;
  if (!xs || !ws) return mxq_set_error(MXQ_ERR_INVALID, "null scale pointer");
  if (ws_numel != 1 && ws_numel != N)
    return mxq_set_error(MXQ_ERR_INVALID, "weight scale must have 1 or N=%lld entries, got %lld", (long long)N, (long long)ws_numel);
  GemmArgs g{};
  g.a = a; g.b = b; g.xs = xs; g.ws = ws; g.bias = bias; g.d = d;
  g.M = M; g.N = N; g.K = K; g.ldd = ldd; g.ws_per_channel = ws_numel == N && N != 1;
  hipStream_t st = (hipStream_t)stream;
  switch (out_dtype) {
    case MXQ_DTYPE_F32: return launch_gemm<kEpiDequant, 0>(g, st);
    case MXQ_DTYPE_F16: return launch_gemm<kEpiDequant, 1>(g, st);
    case MXQ_DTYPE_BF16: return launch_gemm<kEpiDequant, 2>(g, st);
    default: return mxq_set_error(MXQ_ERR_UNSUPPORTED, "output dtype code %d", out_dtype);
  }
}

extern "C" int mxq_int8_gemm_dequant_gelu_absmax(const int8_t* a, const int8_t* b, const float* xs,
                                                 const float* ws, int64_t ws_numel,
                                                 const void* bias_bf16, void* h_bf16,
                                                 float* row_absmax, int64_t M, int64_t N,
                                                 int64_t K, int64_t ldh, void* stream) {
  int rc = check_gemm_shape(a, b, h_bf16, M, N, K, ldh);
  if (rc) return rc;
  if (M == 0 || N == 0) return MXQ_OK;
  if (!xs || !ws || !row_absmax) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  if (ws_numel != 1 && ws_numel != N) return mxq_set_error(MXQ_ERR_INVALID, "bad weight scale length");
  GemmArgs g{};
  g.a = a; g.b = b; g.xs = xs; g.ws = ws; g.bias = bias_bf16; g.d = h_bf16; g.row_absmax = row_absmax;
  g.M = M; g.N = N; g.K = K; g.ldd = ldh; g.ws_per_channel = ws_numel == N && N != 1;
  return launch_gemm<kEpiGelu, 2>(g, (hipStream_t)stream);
}
