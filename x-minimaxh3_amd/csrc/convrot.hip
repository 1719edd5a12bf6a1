// ConvRot: regular-Hadamard rotation of each group of G columns, fused with the pre-quantization
// activation and the per-token INT8 quantizer (gfx950).
//
// Reference: activations x_rot = x_grouped @ H_G, H_G = kron(h4, ..., h4) / sqrt(G) with
// h4 = [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],[-1,1,1,1]] (backends/turbo/vendor/comfy_kitchen/
// tensor/int8_utils.py:11-74), applied in int8_linear before the row quantizer
// (CK/backends/eager/quantization.py:1012-1025, 857-875); the activation first
// (CK/backends/_activations.py:40-53). The reference multiplies with torch's CPU matmul, whose
// accumulation order is internal to the library; here the rotated value is the exact product
// rounded once to the input dtype.
//
// Transform: with y = x H, y_j = sum_i x_i prod_t h4[i_t][j_t] over the base-4 digits t of the
// in-group index, so the rotation is one 4-point transform per digit; column k of h4 is all ones
// but -1 in row 3-k, so a quad (x0..x3) becomes y_k = S - 2 x_{3-k}, S = (x0 + x1) + (x2 + x3).
// It runs in float64: every operation is exact while a group's exponent spread is at most 37
// bits, which makes the result the exact product; the fixed operation order (digit 0 first, the
// same association in every lane) makes it reproducible in all other cases.
//
// Layout: a row is cut into 1024-column windows; in a window lane l holds 16 consecutive
// columns, so digits 0 and 1 of the in-group index are inside the lane and digit d >= 2 is lane
// bit pair d-2. Digits 2 and 3 are brought into the lane by a 16 x 16 transpose of each 16-lane
// group through the wave's LDS region and applied there with the same quad step; digits >= 4
// (G >= 1024) exchange with xor shuffles as y_k = (x_k + x_{k^1}) + (x_{k^2} - x_{k^3}) (rotate16
// in act_rot.h). Groups never straddle lanes (G % 16 == 0, or G = 4 with four groups per lane). Up to four
// waves share a row's windows; the rotated row stays in registers while its absmax is reduced
// (through LDS across the row's waves), then it is quantized and stored with 16-byte stores.
//
// RMS adaLN front end (the H3 block's norm before the QKV and fc1 projections,
// h3serve/native_engine/model/kernels.py:7594-7640 with RMSNorm at layers.py:33-48): a first
// pass over the row sums x^2 (float64, then rounded once: mean = fp32(sum) / K), r =
// 1 / sqrt(mean + eps); every element becomes n = bf16((x * r) * w), then the segment's
// modulation in the eager order: y = bf16(bf16(n * bf16(1 + scale[seg])) + shift[seg]).
// y is optionally stored (the rms_adaln output) and then rotated and quantized as above.

#include "act_f16.h"

namespace mxq {

namespace {

constexpr int kMaxWindows = 20;  // 1024-column windows per row: K <= 20480

struct CrArgs {
  const void* x;
  int8_t* q;
  float* scales;
  int64_t rows;
  int K;       // columns of the quantized row (the raw row has 2K for SwiGLU)
  int digits;  // log4(G); 0: no rotation
  int wpr;     // waves per row: 1, 2 or 4 (4 / wpr rows per block)
  // RMS adaLN front end (kMod != kModNone)
  const uint16_t* norm_w;   // [K] bf16
  const uint16_t* mscale;   // [mod_count, ldm] bf16
  const uint16_t* mshift;   // [mod_count, ldm] bf16
  const int32_t* mrows;     // [rows] segment row of each token
  int64_t ldm, mod_count;
  float eps;
  uint16_t* y_out;          // [rows, K] bf16 modulated rows, or null
};

enum { kModNone = 0, kModQuant = 1, kModOnly = 2 };  // kModOnly: store y, no rotation / quantizer

MXQ_DEVICE uint32_t half_of(const v4u* w, int i) {  // bf16 i of 16 packed in two v4u
  const uint32_t word = w[i >> 3][(i >> 1) & 3];
  return (i & 1) ? (word >> 16) : (word & 0xFFFFu);
}

// Layout: a 256-thread block holds 4 / wpr rows, wpr waves per row. Window j of wave w (of its
// row) is window w + j * wpr of the row: 1024 columns, lane l holding columns 16 l .. 16 l + 15.
// All raw loads of a wave are issued first; the rotated (or, for fp32, float) values stay in
// registers until the row's absmax is known, so each element is read once and written once.
// Per-row partial sums and maxima go through LDS, double-buffered by iteration parity so a
// wave that runs ahead never overwrites a slot another wave still reads.
// kOcc: waves per SIMD the register allocation must allow. Three keeps a bf16 row of up to four
// windows per wave in registers (two leave the memory pipeline short of loads in flight); the
// fp32, the five-window and the RMS-front-end four-window forms need more registers than that.
template <int kAct, int kDtype, int kMod, int kNW,
          int kOcc = (kDtype == MXQ_DTYPE_F32 || kNW > 4 || (kMod != kModNone && kNW > 3)) ? 2 : 3>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kOcc))) void convrot_quant_kernel(CrArgs p) {
  constexpr bool kF32 = kDtype == MXQ_DTYPE_F32, kF16 = kDtype == MXQ_DTYPE_F16;
  static_assert(kMod == kModNone || !kF32, "the RMS adaLN front end takes bfloat16 or float16 rows");
  // the 16-bit row dtype's conversion and rounding (bfloat16 or float16)
  auto cvt = [](uint32_t h) { return kF16 ? f16_to_f32(h) : bf16_to_f32(h); };
  auto rnd = [](float f) { return kF16 ? round_f16(f) : round_bf16(f); };
  auto to_bits = [](float f) { return kF16 ? f32_to_f16_bits(f) : f32_to_bf16_bits(f); };
  constexpr int kRawWords = kF32 ? 16 : (kAct == MXQ_ACT_SWIGLU ? 16 : 8);  // dwords per window
  constexpr int kKeepWords = kF32 ? 16 : 8;
  __shared__ uint32_t red_max[2][4];
  __shared__ double red_ss[2][4];
  __shared__ __attribute__((aligned(16))) double tbuf[4 * kTWave];  // rotation transposes, per wave
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wpr = p.wpr, rpb = 4 / wpr;
  const int slot = wave / wpr, wr = wave - slot * wpr;
  const int windows = (p.K + 1023) >> 10;
  const double inv = 1.0 / (double)(1 << p.digits);  // 1/sqrt(G), exact
  const int64_t xstride = kAct == MXQ_ACT_SWIGLU ? 2 * (int64_t)p.K : p.K;
  int it = 0;

  for (int64_t r0 = (int64_t)blockIdx.x * rpb; r0 < p.rows; r0 += (int64_t)gridDim.x * rpb, it ^= 1) {
    const int64_t row = r0 + slot;
    const bool row_on = row < p.rows;
    // ---- raw loads of every window of this wave
    uint32_t raw[kNW][kRawWords];
#pragma unroll
    for (int j = 0; j < kNW; ++j) {
      const int e0 = (wr + j * wpr) * 1024 + lane * 16;
      const bool on = row_on && e0 < p.K;
      if constexpr (kF32) {
        const v4f* src = reinterpret_cast<const v4f*>(reinterpret_cast<const float*>(p.x) + row * p.K + e0);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const v4f f = on ? src[c] : v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int e = 0; e < 4; ++e) raw[j][4 * c + e] = __float_as_uint(f[e]);
        }
      } else {
        const uint16_t* xr = reinterpret_cast<const uint16_t*>(p.x) + row * xstride;
#pragma unroll
        for (int c = 0; c < kRawWords / 4; ++c) {
          const int64_t off = (c < 2 ? 0 : p.K) + e0 + 8 * (c & 1);  // [gate | up] for SwiGLU
          const v4u w = on ? *reinterpret_cast<const v4u*>(xr + off) : v4u{0, 0, 0, 0};
#pragma unroll
          for (int e = 0; e < 4; ++e) raw[j][4 * c + e] = w[e];
        }
      }
    }
    // ---- RMS statistics of the row (RMS adaLN front end)
    float rinv = 0.0f;
    const uint16_t* msc = nullptr;
    const uint16_t* msh = nullptr;
    if constexpr (kMod != kModNone) {
      double ss = 0.0;
#pragma unroll
      for (int j = 0; j < kNW; ++j) {
        double acc = 0.0;  // squares of bf16 / fp16 values are exact in float32; summed in float64
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float lo = cvt(raw[j][e] & 0xFFFFu), hi = cvt(raw[j][e] >> 16);
          acc += (double)(lo * lo) + (double)(hi * hi);
        }
        ss += acc;
      }
      ss = wave_sum_f64(ss);
      if (lane == 0) red_ss[it][wave] = ss;
      __syncthreads();
      double tot = 0.0;
      for (int i = 0; i < wpr; ++i) tot += red_ss[it][slot * wpr + i];
      const float mean = (float)tot / (float)p.K;
      rinv = 1.0f / sqrtf(mean + p.eps);
      int64_t mr = row_on ? p.mrows[row] : 0;
      mr = mr < 0 ? 0 : (mr >= p.mod_count ? p.mod_count - 1 : mr);
      msc = p.mscale + mr * p.ldm;
      msh = p.mshift + mr * p.ldm;
    }
    // ---- activation / modulation, rotation, rounding to the row dtype; absmax
    uint32_t keep[kNW][kKeepWords];
    uint32_t amax = 0;  // |value| bits (f32 rows) or packed |bf16| pairs (bf16 rows)
#pragma unroll
    for (int j = 0; j < kNW; ++j) {
      const int win = wr + j * wpr;
      if (win >= windows) break;  // uniform over the wave
      const int e0 = win * 1024 + lane * 16;
      const bool on = row_on && e0 < p.K;
      double v[16];
      if constexpr (kF32) {
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = (double)__uint_as_float(raw[j][i]);
      } else {
        const v4u* rw = reinterpret_cast<const v4u*>(raw[j]);
        v4u nw[2], sc[2], sh[2];
        if constexpr (kMod != kModNone) {
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            nw[c] = on ? reinterpret_cast<const v4u*>(p.norm_w + e0)[c] : v4u{0, 0, 0, 0};
            sc[c] = on ? reinterpret_cast<const v4u*>(msc + e0)[c] : v4u{0, 0, 0, 0};
            sh[c] = on ? reinterpret_cast<const v4u*>(msh + e0)[c] : v4u{0, 0, 0, 0};
          }
        }
        uint32_t ybits[8];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          uint32_t b = half_of(rw, i);
          if constexpr (kAct == MXQ_ACT_GELU_TANH) b = kF16 ? gelu_f16(b) : gelu_bf16(b);
          if constexpr (kAct == MXQ_ACT_SWIGLU) b = kF16 ? swiglu_f16(b, half_of(rw + 2, i)) : swiglu_bf16(b, half_of(rw + 2, i));
          if constexpr (kMod != kModNone) {
            const float t = rnd(1.0f + cvt(half_of(sc, i)));
            const float n = rnd((cvt(b) * rinv) * cvt(half_of(nw, i)));
            b = to_bits(rnd(n * t) + cvt(half_of(sh, i)));
            if (i & 1) ybits[i >> 1] |= b << 16; else ybits[i >> 1] = b;
          }
          v[i] = (double)(kF16 ? f16_to_f32(b) : bf16_to_f32(b));
        }
        if constexpr (kMod != kModNone) {
          if (p.y_out && on) {
            v4u* dst = reinterpret_cast<v4u*>(p.y_out + row * p.K + e0);
            dst[0] = v4u{ybits[0], ybits[1], ybits[2], ybits[3]};
            dst[1] = v4u{ybits[4], ybits[5], ybits[6], ybits[7]};
          }
          if constexpr (kMod == kModOnly) continue;
        }
      }
      rotate16(v, p.digits, tbuf + wave * kTWave);
      if constexpr (kF32) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float r = (float)(v[i] * inv);
          keep[j][i] = __float_as_uint(r);
          if (on) amax = amax > abs_bits(r) ? amax : abs_bits(r);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t lo = kF16 ? f64_to_f16_bits(v[2 * i] * inv) : f64_to_bf16_bits(v[2 * i] * inv);
          const uint32_t hi = kF16 ? f64_to_f16_bits(v[2 * i + 1] * inv) : f64_to_bf16_bits(v[2 * i + 1] * inv);
          keep[j][i] = lo | (hi << 16);
          if (on) amax = absmax_acc_bf16x2(amax, keep[j][i]);
        }
      }
    }
    if constexpr (kMod == kModOnly) continue;
    // ---- row absmax across the row's waves, scale
    // (|float16| and |bfloat16| both order like their bit patterns, so one integer maximum serves both)
    const uint32_t hmax = max(amax & 0xFFFFu, amax >> 16);
    const float wmax = wave_absmax(kF32 ? amax : (kF16 ? __float_as_uint(f16_to_f32(hmax)) : hmax << 16));
    if (lane == 0) red_max[it][wave] = __float_as_uint(wmax);
    __syncthreads();
    uint32_t rmax = red_max[it][slot * wpr];
    for (int i = 1; i < wpr; ++i) rmax = rmax > red_max[it][slot * wpr + i] ? rmax : red_max[it][slot * wpr + i];
    const float s = row_scale_from_absmax(__uint_as_float(rmax));
    const float r = 1.0f / round_bf16(s);
    // float16 rows divide by the scale rounded to float16 (torch.finfo(float16).tiny if that is 0),
    // one fp32 division rounded to float16, as the generic quantizer does
    float s16 = round_f16(s);
    if (s16 == 0.0f) s16 = 6.103515625e-05f;
    // ---- quantize from registers, 16-byte stores
#pragma unroll
    for (int j = 0; j < kNW; ++j) {
      const int e0 = (wr + j * wpr) * 1024 + lane * 16;
      if (!row_on || e0 >= p.K) continue;
      int qv[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if constexpr (kF32) {
          qv[i] = quant_round_clamp(__uint_as_float(keep[j][i]) / s);
        } else if constexpr (kF16) {
          const uint32_t h = (keep[j][i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
          qv[i] = quant_round_clamp(round_f16(f16_to_f32(h) / s16));
        } else {
          const uint32_t h = (keep[j][i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
          qv[i] = quant_round_clamp(round_bf16(bf16_to_f32(h) * r));
        }
      }
      uint32_t o[4];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        o[c] = (uint32_t)(qv[4 * c] & 0xFF) | ((uint32_t)(qv[4 * c + 1] & 0xFF) << 8) |
               ((uint32_t)(qv[4 * c + 2] & 0xFF) << 16) | ((uint32_t)(qv[4 * c + 3] & 0xFF) << 24);
      *reinterpret_cast<v4u*>(p.q + row * p.K + e0) = v4u{o[0], o[1], o[2], o[3]};
    }
    if (row_on && wr == 0 && lane == 0) p.scales[row] = s;
  }
}

// Waves per row and windows per wave for a row of K columns.
void row_split(int64_t K, int& wpr, int& nw) {
  const int windows = (int)((K + 1023) / 1024);
  wpr = windows >= 4 ? 4 : (windows >= 2 ? 2 : 1);
  nw = (windows + wpr - 1) / wpr;
}

template <int kAct, int kDtype, int kMod>
int launch_convrot(const CrArgs& a, int nw, hipStream_t st) {
  const int rpb = 4 / a.wpr;
  const unsigned grid = (unsigned)std::min<int64_t>((a.rows + rpb - 1) / rpb, 1 << 20);
  switch (nw) {
    case 1: convrot_quant_kernel<kAct, kDtype, kMod, 1><<<grid, 256, 0, st>>>(a); break;
    case 2: convrot_quant_kernel<kAct, kDtype, kMod, 2><<<grid, 256, 0, st>>>(a); break;
    case 3: convrot_quant_kernel<kAct, kDtype, kMod, 3><<<grid, 256, 0, st>>>(a); break;
    case 4: convrot_quant_kernel<kAct, kDtype, kMod, 4><<<grid, 256, 0, st>>>(a); break;
    case 5: convrot_quant_kernel<kAct, kDtype, kMod, 5><<<grid, 256, 0, st>>>(a); break;
    default: return mxq_set_error(MXQ_ERR_UNSUPPORTED, "row too wide");
  }
  return mxq_check_launch("convrot_quant_kernel");
}

// ---- unit form: bfloat16 rows, G <= 256, K a multiple of 256 ----
// A unit is 256 consecutive columns of a row, held by 16 lanes (16 columns each), so every group
// of G <= 256 columns lies inside one unit (digits 0 and 1 in the lane, digits 2 and 3 across the
// 16 lanes, rotate16). A 16-lane group takes kNU units of one row (units g, g + gr, g + 2 gr, ...,
// so the groups of a wave read adjacent units), and a block holds rpb rows of gr groups each; the
// launcher picks kNU, gr and rpb so that few lanes idle whatever K is (the window form above
// leaves a third of its lanes idle at K = 5376), preferring small blocks (at most 4 waves: at
// 720p 4-wave blocks beat 8- and 16-wave ones by 15-35 %). A row's statistics (absmax, and the RMS
// sum for the adaLN front end) are reduced over its 16 lanes by shuffles and over its groups
// through LDS, double-buffered by iteration parity. The value path is the window form's, with
// the float64 -> bfloat16 rounding done in pairs (the midpoint correction of f64_to_bf16_bits
// runs only for a unit where some float32 value lands on a bfloat16 midpoint) and rows whose
// absmax is finite quantized by the finite-row path.
// A launch of at most 8 rows (one token's row: the M = 1 linear, decode) is bound by the latency
// of one row's work, not by throughput: it takes the fewest units per group, one unit a group in
// blocks of up to kUnitLatWaves waves (K = 5376: 21 groups in 6 waves; the kernel 5.4 -> 3.8 us,
// near the ~3.4 us of an empty launch, against 3 units a group in 2 waves).
constexpr int kUnitMaxWaves = 4;
constexpr int kUnitLatWaves = 6;

// The rotation of one unit up to the transposed layout: digits 0 and 1 in the lane; for
// kDigits >= 3 each 16-lane group transposes its 16 x 16 float64 values through its LDS region
// (as rotate16) and applies digits 2 (and 3) in the lane, leaving lane s of the group with the
// values of columns 16 l + s, l = 0..15. The operations and their order are rotate16's.
template <int kDigits>
MXQ_DEVICE void rotate_unit_fwd(double* v, double* tb) {
  if constexpr (kDigits >= 1) {
#pragma unroll
    for (int j = 0; j < 16; j += 4) h4_quad(v[j], v[j + 1], v[j + 2], v[j + 3]);
  }
  if constexpr (kDigits >= 2) {
#pragma unroll
    for (int j = 0; j < 4; ++j) h4_quad(v[j], v[j + 4], v[j + 8], v[j + 12]);
  }
  if constexpr (kDigits >= 3) {
    const int lane = threadIdx.x & 63, s = lane & 15;
    double* gb = tb + (lane >> 4) * kTGroup;
    typedef double d2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int c = 0; c < 8; ++c) *reinterpret_cast<d2*>(gb + s * kTRow + 2 * c) = d2{v[2 * c], v[2 * c + 1]};
    wave_lds_fence();
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = gb[r * kTRow + s];
    wave_lds_fence();
#pragma unroll
    for (int j = 0; j < 16; j += 4) h4_quad(v[j], v[j + 1], v[j + 2], v[j + 3]);  // digit 2
    if constexpr (kDigits >= 4) {
#pragma unroll
      for (int j = 0; j < 4; ++j) h4_quad(v[j], v[j + 4], v[j + 8], v[j + 12]);  // digit 3
    }
  }
}

// The way back for the rounded values: lane s of a group holds bf16 pairs of columns
// (16 l + s), l = 0..15 (pair m: l = 2m, 2m + 1). It writes each value as 16 bits to row l,
// column s of a 16 x 16 matrix (rows of 48 bytes, groups 800 bytes apart, so that both the
// 16-bit writes and the row reads spread over the banks), and lane l reads its row back as two
// 16-byte loads: columns 16 l .. 16 l + 15 as pairs again. 16-bit traffic, a quarter of a
// float64 transpose. (Scattered 16-bit writes rather than 16-bit loads into register halves:
// with SRAM ECC those loads do not preserve the other half.)
constexpr int kBRow = 48, kBGroup = 800;

MXQ_DEVICE void unit_back16(uint32_t (&w)[8], double* tb) {
  const int lane = threadIdx.x & 63, s = lane & 15;
  char* gb = reinterpret_cast<char*>(tb) + (lane >> 4) * kBGroup;
  wave_lds_fence();  // the float64 transpose of this region has been read
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    reinterpret_cast<uint16_t*>(gb + (2 * m) * kBRow)[s] = (uint16_t)(w[m] & 0xFFFFu);
    reinterpret_cast<uint16_t*>(gb + (2 * m + 1) * kBRow)[s] = (uint16_t)(w[m] >> 16);
  }
  wave_lds_fence();
  const v4u lo = *reinterpret_cast<const v4u*>(gb + s * kBRow);
  const v4u hi = *reinterpret_cast<const v4u*>(gb + s * kBRow + 16);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    w[e] = lo[e];
    w[4 + e] = hi[e];
  }
  wave_lds_fence();  // read before the region's next writes
}

template <int kAct, int kMod, int kDigits, int kNU, bool kTab = false, int kPreMod = 1, int kWaves = kUnitMaxWaves>
__global__ __launch_bounds__(kWaves * 64) void convrot_units_kernel(CrArgs p, int gr, int rpb) {
  constexpr int kRawWords = kAct == MXQ_ACT_SWIGLU ? 16 : 8;  // dwords per unit and lane
  constexpr double kInv = 1.0 / (double)(1 << kDigits);     // 1/sqrt(G), exact
  __shared__ uint32_t red_max[2][4 * kWaves];
  __shared__ double red_ss[2][4 * kWaves];
  extern __shared__ __attribute__((aligned(16))) double tbuf[];  // kTWave per wave of the block
  const int wave = threadIdx.x >> 6;
  const int grp = threadIdx.x >> 4, gl = threadIdx.x & 15;
  const int slot = grp / gr, gi = grp - slot * gr;
  const int units = p.K >> 8;
  const int64_t xstride = kAct == MXQ_ACT_SWIGLU ? 2 * (int64_t)p.K : p.K;
  double* tb = tbuf + wave * kTWave;
  int it = 0;
  // Raw loads of every unit of this group for the batch starting at r, through one raw buffer
  // over rows r .. (the batch's rows span at most 16 * 2 * 2^16 bytes): units past the row and
  // rows past the end pass an offset beyond the buffer and read zeros, without a branch.
  auto load_batch = [&](int64_t r, uint32_t (&raw)[kNU][kRawWords]) {
    const int64_t row = r + slot;
    const bool row_on = slot < rpb && row < p.rows;
    const char* base = reinterpret_cast<const char*>(p.x) + r * xstride * 2;
    const int bytes = (int)std::min<int64_t>((p.rows - r) * xstride * 2, 0x7FFFFFF0);
#pragma unroll
    for (int k = 0; k < kNU; ++k) {
      const int u = gi + k * gr;
      const bool on = row_on && u < units;
      const uint32_t off = on ? (uint32_t)((slot * xstride + u * 256 + gl * 16) * 2) : kBufferOff;
#pragma unroll
      for (int c = 0; c < kRawWords / 4; ++c) {
        const v4u w = buffer_load_x4(base, bytes, off + (c < 2 ? 0u : (uint32_t)p.K * 2u) + 16u * (c & 1));
#pragma unroll
        for (int e = 0; e < 4; ++e) raw[k][4 * c + e] = w[e];
      }
    }
  };
  for (int64_t r0 = (int64_t)blockIdx.x * rpb; r0 < p.rows; r0 += (int64_t)gridDim.x * rpb, it ^= 1) {
    const int64_t row = r0 + slot;
    const bool row_on = slot < rpb && row < p.rows;
    uint32_t raw[kNU][kRawWords];
    load_batch(r0, raw);
    // ---- RMS adaLN front end: the row's segment, then the norm weight, scale and shift words of
    // the first kPreMod units, requested with the raw loads so that their latency overlaps the
    // row sum instead of following it; the other units' words are requested one unit ahead of
    // their use. (All units up front: 144 -> 188 VGPRs at three units, and at the occupancy that
    // leaves, 0.71 -> 0.83 ms for [75600, 5376]; the first unit alone: 0.70 ms.) The loads are
    // unconditional: a unit past the row reads columns 0 .. 15 of a valid row, and its values
    // are left out of the row's absmax and never stored.
    v4u nw[kMod != kModNone ? kNU : 1][2], sc[kMod != kModNone ? kNU : 1][2], sh[kMod != kModNone ? kNU : 1][2];
    const uint16_t* msc = nullptr;
    const uint16_t* msh = nullptr;
    auto load_mod = [&](int k) {
      const int u = gi + k * gr;
      const bool on = row_on && u < units;
      const int e0 = on ? u * 256 + gl * 16 : 0;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        nw[k][c] = reinterpret_cast<const v4u*>(p.norm_w + e0)[c];
        sc[k][c] = reinterpret_cast<const v4u*>(msc + e0)[c];
        sh[k][c] = reinterpret_cast<const v4u*>(msh + e0)[c];
      }
    };
    if constexpr (kMod != kModNone) {
      int64_t mr = row_on ? p.mrows[row] : 0;
      mr = mr < 0 ? 0 : (mr >= p.mod_count ? p.mod_count - 1 : mr);
      msc = p.mscale + mr * p.ldm;
      msh = p.mshift + mr * p.ldm;
#pragma unroll
      for (int k = 0; k < kPreMod; ++k) load_mod(k);
    }
    // ---- RMS statistic of the row (RMS adaLN front end): squares of bf16 values are exact in
    // float64, as are their sums (row-independent of the order while the spread allows)
    float rinv = 0.0f;
    if constexpr (kMod != kModNone) {
      double ss = 0.0;
#pragma unroll
      for (int k = 0; k < kNU; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const double lo = (double)bf16_lo(raw[k][e]), hi = (double)bf16_hi(raw[k][e]);
          ss = __builtin_fma(lo, lo, ss);
          ss = __builtin_fma(hi, hi, ss);
        }
      ss = row16_sum_f64(ss);
      if (gl == 0) red_ss[it][grp] = ss;
      __syncthreads();
      // lane i of each group takes partials i and i + 16 of its row, then the 16 lanes combine
      double tot = 0.0;
      if (slot < rpb)  // groups past the block's rows read no partials
        for (int i = gl; i < gr; i += 16) tot += red_ss[it][slot * gr + i];
      tot = row16_sum_f64(tot);
      const float mean = (float)tot / (float)p.K;
      rinv = 1.0f / sqrtf(mean + p.eps);
    }
    // ---- activation / modulation, rotation, rounding to bf16 pairs; absmax
    uint32_t keep[kNU][8];
    uint32_t amax = 0;  // packed |bf16| pairs
#pragma unroll
    for (int k = 0; k < kNU; ++k) {
      const int u = gi + k * gr;
      const bool on = row_on && u < units;
      const int e0 = u * 256 + gl * 16;
      const v4u* rw = reinterpret_cast<const v4u*>(raw[k]);
      double v[16];
      if constexpr (kMod != kModNone) {
        if (k + 1 >= kPreMod && k + 1 < kNU) load_mod(k + 1);
        uint32_t ybits[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t xw = rw[i >> 2][i & 3], ww = nw[k][i >> 2][i & 3];
          const uint32_t sw = sc[k][i >> 2][i & 3], hw = sh[k][i >> 2][i & 3];
          // t = bf16(1 + scale), n = bf16((x * r) * w), y = bf16(bf16(n * t) + shift), each
          // rounding kept in fp32 form (round_bf16), the pair packed only for the y store
          // (with kTab the words are already bf16(1 + scale), built once per call)
          const float tl = kTab ? bf16_lo(sw) : round_bf16(1.0f + bf16_lo(sw));
          const float th = kTab ? bf16_hi(sw) : round_bf16(1.0f + bf16_hi(sw));
          const float nl = round_bf16((bf16_lo(xw) * rinv) * bf16_lo(ww));
          const float nh = round_bf16((bf16_hi(xw) * rinv) * bf16_hi(ww));
          const float yl = round_bf16(round_bf16(nl * tl) + bf16_lo(hw));
          const float yh = round_bf16(round_bf16(nh * th) + bf16_hi(hw));
          ybits[i] = pair_of_rounded(yl, yh);
          v[2 * i] = (double)yl;
          v[2 * i + 1] = (double)yh;
        }
        if (p.y_out && on) {
          v4u* dst = reinterpret_cast<v4u*>(p.y_out + row * p.K + e0);
          dst[0] = v4u{ybits[0], ybits[1], ybits[2], ybits[3]};
          dst[1] = v4u{ybits[4], ybits[5], ybits[6], ybits[7]};
        }
        if constexpr (kMod == kModOnly) continue;
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          uint32_t b = half_of(rw, i);
          if constexpr (kAct == MXQ_ACT_GELU_TANH) b = gelu_bf16(b);
          if constexpr (kAct == MXQ_ACT_SWIGLU) b = swiglu_bf16(b, half_of(rw + 2, i));
          v[i] = (double)bf16_to_f32(b);
        }
      }
      rotate_unit_fwd<kDigits>(v, tb);
      bool mid = false;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float a = (float)(v[2 * i] * kInv), b = (float)(v[2 * i + 1] * kInv);
        keep[k][i] = pack_bf16x2(a, b);
        mid |= ((__float_as_uint(a) & 0xFFFFu) == 0x8000u) | ((__float_as_uint(b) & 0xFFFFu) == 0x8000u);
      }
      if (mid) {  // a float32 on a bfloat16 midpoint: the exact value decides (f64_to_bf16_bits)
#pragma unroll
        for (int i = 0; i < 8; ++i)
          keep[k][i] = f64_to_bf16_bits(v[2 * i] * kInv) | (f64_to_bf16_bits(v[2 * i + 1] * kInv) << 16);
      }
      uint32_t ua = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) ua = absmax_acc_bf16x2(ua, keep[k][i]);
      amax = on ? absmax_acc_bf16x2(amax, ua) : amax;
      if constexpr (kDigits >= 3) unit_back16(keep[k], tb);
    }
    if constexpr (kMod == kModOnly) continue;
    // ---- row absmax over the group's lanes, then over the row's groups
    const uint32_t bits = row16_max_u32(absmax_bits_of_bf16x2(amax));
    if (gl == 0) red_max[it][grp] = bits;
    __syncthreads();
    uint32_t rmax = 0;
    if (slot < rpb)
      for (int i = gl; i < gr; i += 16) rmax = max(rmax, red_max[it][slot * gr + i]);
    rmax = row16_max_u32(rmax);
    const float amaxf = __uint_as_float(rmax);
    const float s = row_scale_from_absmax(amaxf);
    const float r = 1.0f / round_bf16(s);
    // ---- quantize from registers, 16-byte stores
    auto store_units = [&](auto finite) {
#pragma unroll
      for (int k = 0; k < kNU; ++k) {
        const int u = gi + k * gr;
        if (u >= units) continue;
        const v4u* kw = reinterpret_cast<const v4u*>(keep[k]);
        const v2u o0 = decltype(finite)::value ? quant8_bf16_finite(kw[0], r) : quant8_bf16(kw[0], r);
        const v2u o1 = decltype(finite)::value ? quant8_bf16_finite(kw[1], r) : quant8_bf16(kw[1], r);
        *reinterpret_cast<v4u*>(p.q + row * p.K + u * 256 + gl * 16) = v4u{o0[0], o0[1], o1[0], o1[1]};
      }
    };
    if (row_on) {
      if (finite_absmax(amaxf))
        store_units(std::true_type{});
      else
        store_units(std::false_type{});
    }
    if (row_on && gi == 0 && gl == 0) p.scales[row] = s;
  }
}

// Units per group, groups per row and rows per block for a row of K = 256 * units columns: the
// choice with the fewest idle unit slots in blocks of at most kUnitMaxWaves waves, then the one
// with fewer units per group (fewer registers).
struct UnitSplit {
  int nu, gr, rpb, waves;
};

UnitSplit unit_split(int units) {
  UnitSplit best{0, 0, 0, 0};
  double best_util = -1.0;
  for (int nu = 1; nu <= 4; ++nu) {
    const int gr = (units + nu - 1) / nu;
    if (gr > 4 * kUnitMaxWaves) continue;
    for (int rpb = 1; rpb * gr <= 4 * kUnitMaxWaves; ++rpb) {
      const int waves = (rpb * gr + 3) / 4;
      const double util = (double)(rpb * units) / (double)(waves * 4 * nu);
      if (util > best_util + 1e-9 || (util > best_util - 1e-9 && waves < best.waves)) {
        best_util = util;
        best = UnitSplit{nu, gr, rpb, waves};
      }
    }
  }
  return best;
}

template <int kAct, int kMod, int kDigits, bool kTab = false>
int launch_units(const CrArgs& a, const UnitSplit& u, hipStream_t st) {
  // One row batch per block (measured faster at 720p than persistent blocks that prefetch the
  // next batch); small blocks, many resident per CU, hide the load latency instead.
  const unsigned grid = (unsigned)std::min<int64_t>((a.rows + u.rpb - 1) / u.rpb, 1 << 20);
  const unsigned threads = (unsigned)(u.waves * 64);
  const size_t lds = (size_t)u.waves * kTWave * sizeof(double);
  if (u.waves > kUnitMaxWaves) {  // the few-row split: one unit a group
    convrot_units_kernel<kAct, kMod, kDigits, 1, kTab, 1, kUnitLatWaves><<<grid, threads, lds, st>>>(a, u.gr, u.rpb);
    return mxq_check_launch("convrot_units_kernel");
  }
  switch (u.nu) {
    case 1: convrot_units_kernel<kAct, kMod, kDigits, 1, kTab><<<grid, threads, lds, st>>>(a, u.gr, u.rpb); break;
    case 2: convrot_units_kernel<kAct, kMod, kDigits, 2, kTab><<<grid, threads, lds, st>>>(a, u.gr, u.rpb); break;
    case 3: convrot_units_kernel<kAct, kMod, kDigits, 3, kTab><<<grid, threads, lds, st>>>(a, u.gr, u.rpb); break;
    default: convrot_units_kernel<kAct, kMod, kDigits, 4, kTab><<<grid, threads, lds, st>>>(a, u.gr, u.rpb); break;
  }
  return mxq_check_launch("convrot_units_kernel");
}

template <int kAct, int kMod, bool kTab = false>
int launch_units_digits(const CrArgs& a, hipStream_t st) {
  UnitSplit u = unit_split(a.K >> 8);
  if (a.rows <= 8) {  // latency-bound: fewest units per group, one row a block
    const int units = (int)(a.K >> 8);
    if (units <= 4 * kUnitLatWaves) {
      u = UnitSplit{1, units, 1, (units + 3) / 4};
    } else {
      for (int nu = 1; nu <= 4; ++nu) {
        const int gr = (units + nu - 1) / nu;
        if (gr <= 4 * kUnitMaxWaves) { u = UnitSplit{nu, gr, 1, (gr + 3) / 4}; break; }
      }
    }
  }
  switch (a.digits) {
    case 0: return launch_units<kAct, kMod, 0, kTab>(a, u, st);
    case 1: return launch_units<kAct, kMod, 1, kTab>(a, u, st);
    case 2: return launch_units<kAct, kMod, 2, kTab>(a, u, st);
    case 3: return launch_units<kAct, kMod, 3, kTab>(a, u, st);
    default: return launch_units<kAct, kMod, 4, kTab>(a, u, st);
  }
}

// The unit form takes bf16 rows with G <= 256 and K a multiple of 256 up to 4 * 32 units.
bool units_fit(int64_t cols, int digits) { return digits <= 4 && cols % 256 == 0 && cols <= 256 * 4 * 4 * kUnitMaxWaves; }

__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
                                                      int64_t rows, int64_t cols) {
  const int64_t n = rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / cols, c = i - r * cols;
    y[i] = (uint16_t)swiglu_bf16(x[r * 2 * cols + c], x[r * 2 * cols + cols + c]);
  }
}

// t[m, c] = bf16(1 + scale[m, c]) for the modulation rows (c < cols, row stride ld): the factor
// every token of segment m multiplies its normalized value by, formed once per call instead of
// once per token and element. Eight columns (16 bytes) per thread.
__global__ __launch_bounds__(256) void one_plus_rows_kernel(const uint16_t* __restrict__ scale, uint16_t* __restrict__ t,
                                                            int64_t ld, int64_t mod_count, int64_t cols) {
  const int64_t per_row = cols / 8, n = mod_count * per_row;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = i / per_row, c = (i - m * per_row) * 8;
    const v4u w = *reinterpret_cast<const v4u*>(scale + m * ld + c);
    v4u o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = pack_bf16x2(1.0f + bf16_lo(w[e]), 1.0f + bf16_hi(w[e]));
    *reinterpret_cast<v4u*>(t + m * ld + c) = o;
  }
}

}  // namespace
}  // namespace mxq

using namespace mxq;

extern "C" int mxq_quantize_int8_rowwise_convrot(const void* x, int x_dtype, int8_t* q, float* scales,
                                                 int64_t rows, int64_t cols, int64_t group_size,
                                                 int input_act, void* stream) {
  if (rows < 0 || cols < 0) return mxq_set_error(MXQ_ERR_INVALID, "negative shape");
  int digits = 0;
  if (group_size != 0) {
    if (group_size < 4 || (group_size & (group_size - 1)) || __builtin_ctzll((uint64_t)group_size) % 2)
      return mxq_set_error(MXQ_ERR_INVALID, "Regular Hadamard size must be a power of 4, got %lld", (long long)group_size);
    digits = __builtin_ctzll((uint64_t)group_size) / 2;
    if (cols % group_size)
      return mxq_set_error(MXQ_ERR_INVALID, "ConvRot group size %lld does not divide input features %lld",
                           (long long)group_size, (long long)cols);
    if (group_size > 1024) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "ConvRot group size above 1024");
  }
  if (input_act < MXQ_ACT_NONE || input_act > MXQ_ACT_SWIGLU)
    return mxq_set_error(MXQ_ERR_INVALID, "unsupported input_act code %d", input_act);
  if (x_dtype != MXQ_DTYPE_BF16 && x_dtype != MXQ_DTYPE_F16 && !(x_dtype == MXQ_DTYPE_F32 && input_act == MXQ_ACT_NONE))
    return mxq_set_error(MXQ_ERR_UNSUPPORTED, "rotation quantizer takes bfloat16 or float16 (or float32 without an activation)");
  if (rows == 0 || cols == 0) return MXQ_OK;
  if (!x || !q || !scales) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  if (cols % 16) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "columns must be a multiple of 16");
  if ((uintptr_t)x % 16 || (uintptr_t)q % 16) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "x and q must be 16-byte aligned");
  if (cols > (int64_t)kMaxWindows * 1024)
    return mxq_set_error(MXQ_ERR_UNSUPPORTED, "row of %lld columns too wide (max %d)", (long long)cols, kMaxWindows * 1024);
  CrArgs a{x, q, scales, rows, (int)cols, digits};
  int nw = 1;
  row_split(cols, a.wpr, nw);
  hipStream_t st = (hipStream_t)stream;
  if (x_dtype == MXQ_DTYPE_F32) return launch_convrot<MXQ_ACT_NONE, MXQ_DTYPE_F32, kModNone>(a, nw, st);
  if (x_dtype == MXQ_DTYPE_F16) {
    switch (input_act) {
      case MXQ_ACT_NONE: return launch_convrot<MXQ_ACT_NONE, MXQ_DTYPE_F16, kModNone>(a, nw, st);
      case MXQ_ACT_GELU_TANH: return launch_convrot<MXQ_ACT_GELU_TANH, MXQ_DTYPE_F16, kModNone>(a, nw, st);
      default: return launch_convrot<MXQ_ACT_SWIGLU, MXQ_DTYPE_F16, kModNone>(a, nw, st);
    }
  }
  if (units_fit(cols, digits)) {
    switch (input_act) {
      case MXQ_ACT_NONE: return launch_units_digits<MXQ_ACT_NONE, kModNone>(a, st);
      case MXQ_ACT_GELU_TANH: return launch_units_digits<MXQ_ACT_GELU_TANH, kModNone>(a, st);
      default: return launch_units_digits<MXQ_ACT_SWIGLU, kModNone>(a, st);
    }
  }
  switch (input_act) {
    case MXQ_ACT_NONE: return launch_convrot<MXQ_ACT_NONE, MXQ_DTYPE_BF16, kModNone>(a, nw, st);
    case MXQ_ACT_GELU_TANH: return launch_convrot<MXQ_ACT_GELU_TANH, MXQ_DTYPE_BF16, kModNone>(a, nw, st);
    default: return launch_convrot<MXQ_ACT_SWIGLU, MXQ_DTYPE_BF16, kModNone>(a, nw, st);
  }
}

extern "C" int mxq_swiglu_bf16(const void* x, void* y, int64_t rows, int64_t cols, void* stream) {
  if (rows < 0 || cols < 0) return mxq_set_error(MXQ_ERR_INVALID, "negative shape");
  if (rows == 0 || cols == 0) return MXQ_OK;
  if (!x || !y) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  const int64_t n = rows * cols;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 65536);
  swiglu_kernel<<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>((const uint16_t*)x, (uint16_t*)y, rows, cols);
  return mxq_check_launch("swiglu_kernel");
}

static int rms_adaln_launch(const void* x, const void* norm_weight, const void* scale, const void* shift,
                            int64_t ld_mod, int64_t mod_count, const int32_t* mod_rows, float eps, void* y_out,
                            int8_t* q, float* scales, int64_t rows, int64_t cols, int64_t group_size, bool f16,
                            void* workspace, int64_t workspace_bytes, void* stream) {
  if (rows < 0 || cols < 0) return mxq_set_error(MXQ_ERR_INVALID, "negative shape");
  int digits = 0;
  if (q && group_size != 0) {
    if (group_size < 4 || (group_size & (group_size - 1)) || __builtin_ctzll((uint64_t)group_size) % 2)
      return mxq_set_error(MXQ_ERR_INVALID, "Regular Hadamard size must be a power of 4, got %lld", (long long)group_size);
    digits = __builtin_ctzll((uint64_t)group_size) / 2;
    if (cols % group_size)
      return mxq_set_error(MXQ_ERR_INVALID, "ConvRot group size %lld does not divide input features %lld",
                           (long long)group_size, (long long)cols);
    if (group_size > 1024) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "ConvRot group size above 1024");
  }
  if (rows == 0 || cols == 0) return MXQ_OK;
  if (!x || !norm_weight || !scale || !shift || !mod_rows) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  if (!q && !y_out) return mxq_set_error(MXQ_ERR_INVALID, "neither a modulated output nor a quantized output");
  if (q && !scales) return mxq_set_error(MXQ_ERR_INVALID, "null scales");
  if (mod_count < 1 || ld_mod < cols) return mxq_set_error(MXQ_ERR_INVALID, "bad modulation table");
  if (cols % 16 || ld_mod % 8) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "columns and modulation stride must be multiples of 16 and 8");
  if ((uintptr_t)x % 16 || (uintptr_t)q % 16 || (uintptr_t)y_out % 16 || (uintptr_t)norm_weight % 16 ||
      (uintptr_t)scale % 16 || (uintptr_t)shift % 16)
    return mxq_set_error(MXQ_ERR_UNSUPPORTED, "tensors must be 16-byte aligned");
  if (cols > (int64_t)kMaxWindows * 1024)
    return mxq_set_error(MXQ_ERR_UNSUPPORTED, "row of %lld columns too wide (max %d)", (long long)cols, kMaxWindows * 1024);
  CrArgs a{x, q, scales, rows, (int)cols, digits};
  int nw = 1;
  row_split(cols, a.wpr, nw);
  a.norm_w = (const uint16_t*)norm_weight;
  a.mscale = (const uint16_t*)scale;
  a.mshift = (const uint16_t*)shift;
  a.mrows = mod_rows;
  a.ldm = ld_mod;
  a.mod_count = mod_count;
  a.eps = eps;
  a.y_out = (uint16_t*)y_out;
  hipStream_t st = (hipStream_t)stream;
  if (f16) {  // float16 rows: the window form
    if (q) return launch_convrot<MXQ_ACT_NONE, MXQ_DTYPE_F16, kModQuant>(a, nw, st);
    return launch_convrot<MXQ_ACT_NONE, MXQ_DTYPE_F16, kModOnly>(a, nw, st);
  }
  if (units_fit(cols, digits)) {
    if (q && workspace && workspace_bytes >= mod_count * ld_mod * 2 && (uintptr_t)workspace % 16 == 0) {
      // bf16(1 + scale) of every modulation row into the workspace, then the kernel reads it there
      uint16_t* t = (uint16_t*)workspace;
      const int64_t n = mod_count * (cols / 8);
      one_plus_rows_kernel<<<(unsigned)std::min<int64_t>((n + 255) / 256, 4096), 256, 0, st>>>(
          (const uint16_t*)scale, t, ld_mod, mod_count, cols);
      if (int rc = mxq_check_launch("one_plus_rows_kernel")) return rc;
      a.mscale = t;
      return launch_units_digits<MXQ_ACT_NONE, kModQuant, true>(a, st);
    }
    if (q) return launch_units_digits<MXQ_ACT_NONE, kModQuant>(a, st);
    return launch_units_digits<MXQ_ACT_NONE, kModOnly>(a, st);
  }
  if (q) return launch_convrot<MXQ_ACT_NONE, MXQ_DTYPE_BF16, kModQuant>(a, nw, st);
  return launch_convrot<MXQ_ACT_NONE, MXQ_DTYPE_BF16, kModOnly>(a, nw, st);
}

extern "C" int mxq_rms_adaln_quantize_int8(const void* x, const void* norm_weight, const void* scale,
                                           const void* shift, int64_t ld_mod, int64_t mod_count,
                                           const int32_t* mod_rows, float eps, void* y_out, int8_t* q,
                                           float* scales, int64_t rows, int64_t cols, int64_t group_size,
                                           void* workspace, int64_t workspace_bytes, void* stream) {
  if (workspace_bytes < 0) return mxq_set_error(MXQ_ERR_INVALID, "negative workspace size");
  return rms_adaln_launch(x, norm_weight, scale, shift, ld_mod, mod_count, mod_rows, eps, y_out, q, scales, rows,
                          cols, group_size, false, workspace, workspace_bytes, stream);
}

extern "C" int mxq_rms_adaln_quantize_int8_f16(const void* x, const void* norm_weight, const void* scale,
                                               const void* shift, int64_t ld_mod, int64_t mod_count,
                                               const int32_t* mod_rows, float eps, void* y_out, int8_t* q,
                                               float* scales, int64_t rows, int64_t cols, int64_t group_size,
                                               void* stream) {
  return rms_adaln_launch(x, norm_weight, scale, shift, ld_mod, mod_count, mod_rows, eps, y_out, q, scales, rows,
                          cols, group_size, true, nullptr, 0, stream);
}
