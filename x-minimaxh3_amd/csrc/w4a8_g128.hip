// Group-128 W4A8 GEMM with a direct-to-LDS pipeline (gfx950).
//
// y[m, n] = out(facc[m, n] * xs[m]), facc = fma(fp32(P_g), s[g, n], facc) over the 128-wide
// K-groups g in order, P_g = sum over the group of a[m, k] * (c[n, k] - 8) exactly in int32
// (the contract of the general kernel in w4a8.hip; this file is its fast path for group 128).
//
// Two workgroups per CU (a 3-stage ring of 24 KB stages; at most 128 VGPRs per lane of int32
// and fp32 accumulators, all in VGPRs): each SIMD runs two waves, so one wave's per-group fold
// (v_cvt_f32_i32 + v_fma_mix_f32 per accumulator, the fp16 scale converted inside the fma) and
// nibble unpack issue while the other wave's MFMAs execute. With one workgroup per CU the
// accumulators sat in AGPRs and every fold needed an extra v_accvgpr_read: 1.6x slower.
//
// Workgroup: 4 wave64s side by side along N; a 128 x 128 tile, wave w owning channels
// w*32 + [0, 32) of all 128 rows as four v_mfma_i32_32x32x32_i8 blocks (activations first:
// lane l holds channel l % 32, so a lane needs one group scale per group).
//  * One K stage = one group. Each stage's A (kBM rows x 128 B), packed B (128 rows x 64 B) and
//    the group's 128 fp16 scales are fetched with direct-to-LDS buffer loads into a ring of kNS
//    stages, kNS - 1 stages ahead. The lane offsets of the loads are fixed registers and the K
//    advance is a scalar offset, so a load costs no vector instruction; the stage loop is
//    unrolled by kNS, so every LDS read is a fixed base register plus an immediate.
//  * Lane half h = l / 32 consumes k in [64 h, 64 h + 64) of the stage; K-step s the 16 k from
//    64 h + 16 s on both operands (the int32 sum over a group is order-free).
//  * At the start of group g each block's int32 accumulators still hold group g-1's sum; the
//    block is folded into its fp32 accumulators just before its first MFMA of group g, so the
//    fold of one block issues while the previous block's MFMA executes (a wave issues in order:
//    MFMAs issued back to back would leave the VALU work serialised behind them). The scale of
//    group g-1 was read from its stage during group g-1. The next K-step's A fragment reads and
//    nibble unpack are interleaved with the MFMAs the same way.
// LDS rows: A 128 B with chunk c at slot c ^ ((r >> 1) & 7); B 64 B with chunk c at slot
// c ^ ((r >> 2) & 3) -- conflict-free for sixteen consecutive rows read at one chunk.

#include "w4a8_common.h"

namespace mxq {

namespace {

// A workgroup is four waves side by side along N. With 128-row tiles a CU holds two workgroups,
// i.e. two waves per SIMD: one wave's fold and unpack VALU work issues while the other's MFMAs
// run. (A 128 x 256 tile with eight waves per workgroup, a third less L2 -> LDS traffic per MAC,
// measured no faster.) Problems with fewer 128-row tiles than two per CU (M = 512 at N = 10240:
// 320 tiles) run 64-row tiles, three workgroups per CU, so that every CU holds two or three.
constexpr int kBN = 128, kNS = 3;
constexpr int kWaves = kBN / 32;
constexpr int kThreads = kWaves * 64;
constexpr int kStageB = kBN * 64;   // 8 KB packed
constexpr int kScaleBytes = kBN * 2;
constexpr int kBLoads = kStageB / 1024 / kWaves;  // 2
constexpr int kScaleLanes = kScaleBytes / kWaves / 16;  // lanes per wave fetching scales
static_assert(kBLoads * kWaves * 16 == kBN, "load split");

template <int kBM_>
struct W4Cfg {
  static constexpr int kBM = kBM_;
  static constexpr int kBI = kBM / 32;                         // MFMA blocks per wave along M
  static constexpr int kOcc = kBM == 128 ? 2 : 3;              // workgroups per CU
  static constexpr int kStageA = kBM * 128;
  static constexpr int kStage = kStageA + kStageB + kScaleBytes;  // A | packed B | scales
  static constexpr int kLds = kNS * kStage;
  static constexpr int kALoads = kStageA / 1024 / kWaves;      // direct-to-LDS loads per wave per stage
  static constexpr int kLoads = kALoads + kBLoads + 1;         // + the wave's share of the scales
  static_assert(kALoads * kWaves * 8 == kBM, "load split");
  static_assert(kOcc * kLds <= 160 * 1024, "LDS per CU");
  static_assert((kNS - 1) * kStage + (kBI - 1) * 32 * 128 < 65536, "LDS read offsets fit the 16-bit immediate");
};

struct Tile {
  int64_t m0, n0;
};

// An empty asm that takes a block's 16 folded values and claims to rewrite its A fragment. The
// block's first MFMA of a group (zero accumulator input) reads that fragment, so it cannot be
// placed above the fold. Without this the fold, being plain arithmetic, was placed below all
// sixteen MFMAs of the group, and every old accumulator had to be copied out first (32
// v_mov_b64 per group and wave).
MXQ_DEVICE void order_after_fold(v4i& frag, const float (&f)[16]) {
  __asm__ volatile("" : "+v"(frag)
                   : "v"(f[0]), "v"(f[1]), "v"(f[2]), "v"(f[3]), "v"(f[4]), "v"(f[5]), "v"(f[6]), "v"(f[7]),
                     "v"(f[8]), "v"(f[9]), "v"(f[10]), "v"(f[11]), "v"(f[12]), "v"(f[13]), "v"(f[14]), "v"(f[15]));
}

template <int kBM>
MXQ_DEVICE Tile tile_of(const W4Args& p) {
  const int num = p.tiles_m * p.tiles_n, per = num / 8, bid = blockIdx.x;
  const int t = bid < per * 8 ? (bid % 8) * per + bid / 8 : bid;  // XCD-contiguous ranges
  const int group = 8 * p.tiles_n, g = t / group, first = g * 8;
  const int gm = min(p.tiles_m - first, 8), in = t % group;
  return Tile{(int64_t)(first + in % gm) * kBM, (int64_t)(in / gm) * kBN};
}

// A 16-bit LDS read issued as inline assembly, like lds_read_b128 (its wait is placed by hand).
template <int kOff>
MXQ_DEVICE uint32_t lds_read_u16(uint32_t addr) {
  uint32_t r;
  __asm__ volatile("ds_read_u16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(kOff));
  return r;
}

template <int kOut, bool kPrepared, int kTileM>
__global__ __launch_bounds__(kThreads, W4Cfg<kTileM>::kOcc) void w4a8_g128_kernel(W4Args p) {
  typedef W4Cfg<kTileM> C;
  constexpr int kBM = C::kBM, kBI = C::kBI, kStageA = C::kStageA, kStage = C::kStage, kLds = C::kLds;
  constexpr int kALoads = C::kALoads, kLoads = C::kLoads;
  __shared__ __attribute__((aligned(16))) char lds[kLds];

  const Tile tile = tile_of<kBM>(p);
  const int64_t m0 = tile.m0, n0 = tile.n0;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(wave);  // scalar: LDS destinations are scalar arithmetic
  const int lr = lane & 31, lh = lane >> 5;
  const int64_t khalf = p.K / 2;
  const int ktiles = (int)(p.K / 128);

  // ---- direct-to-LDS sources: raw buffers over A, the packed weights and the scales (the
  // launcher guarantees each spans fewer than 2^31 bytes), a fixed 32-bit byte offset per lane
  // and load, and the K advance as the scalar offset.
  const int a_bytes = (int)(p.M * p.K), b_bytes = (int)(p.N * khalf), s_bytes = (int)(p.N * ktiles * 2);
  uint32_t a_off[kALoads], b_off[kBLoads];
#pragma unroll
  for (int t = 0; t < kALoads; ++t) {
    const int r = (wave * kALoads + t) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    a_off[t] = (uint32_t)(min(m0 + r, p.M - 1) * p.K + c * 16);
  }
#pragma unroll
  for (int t = 0; t < kBLoads; ++t) {
    const int r = (wave * kBLoads + t) * 16 + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 2) & 3);
    b_off[t] = (uint32_t)(min(n0 + r, p.N - 1) * khalf + c * 16);
  }
  // wave w fetches scale bytes [64 w, 64 w + 64) of the group's row of kBN (16 per lane).
  const int64_t s_col = n0 + wave * 32 + lane * 8;
  const uint32_t s_off = (uint32_t)((s_col < p.N ? s_col : 0) * 2);

  // Stage kt into ring slot kSlot (= kt % kNS).
  auto issue_stage = [&](int kt, auto SlotC) {
    constexpr int kSlot = decltype(SlotC)::value;
    char* st = lds + kSlot * kStage;
    const int ka = kt * 128, kb = kt * 64, ksc = kt * (int)p.N * 2;
#pragma unroll
    for (int t = 0; t < kALoads; ++t)
      buffer_load_lds16(p.a, a_bytes, (lptr_t)(st + (wv * kALoads + t) * 1024), a_off[t], ka);
#pragma unroll
    for (int t = 0; t < kBLoads; ++t)
      buffer_load_lds16(p.w, b_bytes, (lptr_t)(st + kStageA + (wv * kBLoads + t) * 1024), b_off[t], kb);
    if (lane < kScaleLanes)
      buffer_load_lds16(p.gs, s_bytes, (lptr_t)(st + kStageA + kStageB + wv * (kScaleBytes / kWaves)), s_off, ksc);
  };

  v16i acc[kBI];
  float facc[kBI][16];
#pragma unroll
  for (int i = 0; i < kBI; ++i) {
    acc[i] = v16i{};
#pragma unroll
    for (int r = 0; r < 16; ++r) facc[i][r] = 0.0f;
  }

  // LDS read bases (the ring slot and the block are immediates): A for K-steps 0..3, the two B
  // chunks, and this lane's channel scale.
  const uint32_t lds_addr = (uint32_t)(uintptr_t)(lptr_t)lds;
  const int a_f = (lr >> 1) & 7;
  uint32_t a_base[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) a_base[s] = lds_addr + (uint32_t)lr * 128 + (uint32_t)(((lh * 4 + s) ^ a_f) << 4);
  const int b_f = (lr >> 2) & 3;
  const uint32_t b_row = lds_addr + (uint32_t)kStageA + (uint32_t)(wave * 32 + lr) * 64;
  const uint32_t b_base0 = b_row + (uint32_t)(((2 * lh) ^ b_f) << 4);
  const uint32_t b_base1 = b_row + (uint32_t)(((2 * lh + 1) ^ b_f) << 4);
  const int s_idx = wave * 32 + lr;  // this lane's channel within the tile
  const uint32_t s_base = lds_addr + (uint32_t)(kStageA + kStageB + s_idx * 2);

  issue_stage(0, std::integral_constant<int, 0>{});
  if (ktiles > 1) {
    issue_stage(1, std::integral_constant<int, 1>{});
    wait_vmcnt<kLoads>();
  } else {
    wait_vmcnt<0>();
  }
  barrier_no_drain();

  auto unpack_step = [&](const v4i (&bq)[2], int s) {
    uint32_t o0, o1, o2, o3;
    if constexpr (kPrepared) {
      unpack8_prepared((uint32_t)bq[s >> 1][(s & 1) * 2], o0, o1);
      unpack8_prepared((uint32_t)bq[s >> 1][(s & 1) * 2 + 1], o2, o3);
    } else {
      unpack8((uint32_t)bq[s >> 1][(s & 1) * 2], o0, o1);
      unpack8((uint32_t)bq[s >> 1][(s & 1) * 2 + 1], o2, o3);
    }
    return v4i{(int)o0, (int)o1, (int)o2, (int)o3};
  };

  float sc = 0.0f;  // scale of the previous group; zero before the first (an exact no-op fold of zeros)
  // One stage = group kt, in ring slot kSlot = kt % kNS. At K-step 0, block i's accumulators
  // still hold group kt-1's sum: they are folded (16 x cvt + fma) right before block i's first
  // MFMA of group kt, so each fold issues while the previous block's MFMA executes. The A
  // fragment of block i for K-step s+1 is read right after block i's MFMA of step s; the next
  // step's nibble unpack follows the second MFMA of each step.
  auto stage = [&](int kt, auto SlotC) {
    constexpr int kSlot = decltype(SlotC)::value;
    constexpr int so = kSlot * kStage;
    v4i bq[2];
    bq[0] = lds_read_b128<so>(b_base0);
    bq[1] = lds_read_b128<so>(b_base1);
    v4i fa[kBI];
    static_for<kBI>([&](auto I) { fa[decltype(I)::value] = lds_read_b128<so + decltype(I)::value * 32 * 128>(a_base[0]); });
    const uint32_t sraw = lds_read_u16<so>(s_base);  // this group's scale, folded during the next group
    if (kt + kNS - 1 < ktiles) issue_stage(kt + kNS - 1, std::integral_constant<int, (kSlot + kNS - 1) % kNS>{});
    wait_lgkm<0>();
    __builtin_amdgcn_sched_barrier(0);
    v4i fb = unpack_step(bq, 0);
    static_for<4>([&](auto S) {
      constexpr int s = decltype(S)::value;
      v4i fb_next;
      // The wave folding its accumulators (K-step 0, VALU-dense) issues ahead of the other wave
      // on its SIMD, which is then in its MFMA-dense K-steps: 2 % faster than equal priorities
      // (priority raised around each MFMA, or for K-steps 1-3 instead, measured no faster).
      if constexpr (s == 0) __builtin_amdgcn_s_setprio(1);
      if constexpr (s == 1) __builtin_amdgcn_s_setprio(0);
      static_for<kBI>([&](auto I) {
        constexpr int i = decltype(I)::value;
        if constexpr (s == 0) {
#pragma unroll
          for (int r = 0; r < 16; ++r) facc[i][r] = fmaf((float)acc[i][r], sc, facc[i][r]);
          order_after_fold(fa[i], facc[i]);
        } else {
          // block i's fragment of this step was read after its previous MFMA; the reads of the
          // later blocks may still be in flight
          wait_lgkm<kBI - 1 - i>();
        }
        __builtin_amdgcn_sched_barrier(0);
        acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb, s == 0 ? v16i{} : acc[i], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (s < 3) fa[i] = lds_read_b128<so + i * 32 * 128>(a_base[s + 1]);
        if constexpr (i == 1 && s < 3) fb_next = unpack_step(bq, s + 1);
        __builtin_amdgcn_sched_barrier(0);
      });
      if constexpr (s < 3) fb = fb_next;
    });
    sc = f16_to_f32((uint16_t)sraw);
    // Stage kt+1 has landed (later stages may stay in flight); slot kSlot is free.
    if (kt + kNS - 1 < ktiles)
      wait_vmcnt<(kNS - 2) * kLoads>();
    else if (kt + kNS - 2 < ktiles)
      wait_vmcnt<(kNS - 3) * kLoads>();
    else
      wait_vmcnt<0>();
    wait_lgkm<0>();
    __builtin_amdgcn_sched_barrier(0);
    barrier_no_drain();
  };

  static_assert(kNS == 3, "the stage loop is unrolled by the ring depth");
  int kt = 0;
  for (; kt + kNS <= ktiles; kt += kNS) {
    stage(kt, std::integral_constant<int, 0>{});
    stage(kt + 1, std::integral_constant<int, 1>{});
    stage(kt + 2, std::integral_constant<int, 2>{});
  }
  if (kt < ktiles) stage(kt, std::integral_constant<int, 0>{});
  if (kt + 1 < ktiles) stage(kt + 1, std::integral_constant<int, 1>{});
#pragma unroll
  for (int i = 0; i < kBI; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) facc[i][r] = fmaf((float)acc[i][r], sc, facc[i][r]);

  // ---- epilogue: y = out(facc * (xs / 16)); y = out(y + bias). The main loop's last barrier
  // left the LDS free: the tile's row scales go there first (every global read of the
  // epilogue is done before its first store, so no store can delay a later load), then the
  // output tile, which is written back as 16-byte row chunks.
  typedef typename OutT<kOut>::T OT;
  constexpr int kE = sizeof(OT);
  constexpr int kPitch = kBN * kE + 16;  // padded row: the two half-waves' rows hit different banks
  static_assert(128 * 4 + kBM * kPitch <= kLds, "epilogue staging exceeds the LDS allocation");
  float* s_xs = reinterpret_cast<float*>(lds);
  char* s_out = lds + 128 * 4;
  const OT* bias = reinterpret_cast<const OT*>(p.bias);
  const int64_t col = n0 + s_idx;
  const float bv = bias ? OutT<kOut>::load(bias + min(col, p.N - 1)) : -0.0f;
  if (threadIdx.x < kBM) s_xs[threadIdx.x] = p.xs[min(m0 + threadIdx.x, p.M - 1)] * 0.0625f;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kBI; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = i * 32 + (r >> 2) * 8 + lh * 4 + (r & 3);
      const float y = OutT<kOut>::round(facc[i][r] * s_xs[row]);
      const float yb = y + bv;
      if constexpr (kE == 4) {
        *reinterpret_cast<float*>(s_out + row * kPitch + s_idx * 4) = yb;
      } else {
        const uint16_t h = kOut == 1 ? (uint16_t)f32_to_f16_bits(yb) : (uint16_t)f32_to_bf16_bits(yb);
        *reinterpret_cast<uint16_t*>(s_out + row * kPitch + s_idx * 2) = h;
      }
    }
  }
  __syncthreads();
  constexpr int kChunksRow = kBN * kE / 16;
  constexpr int kPerElem = 16 / kE;
  char* D = reinterpret_cast<char*>(p.d);
  const bool vec = ((uintptr_t)p.d % 16 == 0) && ((p.ldd * kE) % 16 == 0);
#pragma unroll
  for (int q = 0; q < kBM * kChunksRow / kThreads; ++q) {
    const int id = q * kThreads + threadIdx.x;
    const int row = id / kChunksRow, ch = id % kChunksRow;
    const int64_t grow = m0 + row, gcol = n0 + ch * kPerElem;
    if (grow >= p.M) continue;
    const v4u v = *reinterpret_cast<const v4u*>(s_out + row * kPitch + ch * 16);
    char* dst = D + (grow * p.ldd + gcol) * kE;
    if (vec && gcol + kPerElem <= p.N) {  // nontemporal: 8192 x 5120 x 5120 0.252 -> 0.250 ms
      __builtin_nontemporal_store(v, reinterpret_cast<v4u*>(dst));
    } else {
      // Element by element from the register words (taking the address of v would place it in
      // memory, and the compiler then moves such per-thread arrays into LDS).
#pragma unroll
      for (int e = 0; e < kPerElem; ++e) {
        if (gcol + e < p.N) {
          const uint32_t word = v[e * kE / 4];
          if constexpr (kE == 4)
            *reinterpret_cast<uint32_t*>(dst + e * 4) = word;
          else
            *reinterpret_cast<uint16_t*>(dst + e * 2) = (uint16_t)(word >> (16 * (e & 1)));
        }
      }
    }
  }
}

template <int kBM>
int launch_tiles(W4Args p, int out_dtype, bool prepared, hipStream_t st) {
  p.tiles_m = (int)((p.M + kBM - 1) / kBM);
  p.tiles_n = (int)((p.N + kBN - 1) / kBN);
  const unsigned grid = (unsigned)(p.tiles_m * p.tiles_n);
  switch (out_dtype * 2 + (prepared ? 1 : 0)) {
    case MXQ_DTYPE_F32 * 2: w4a8_g128_kernel<0, false, kBM><<<grid, kThreads, 0, st>>>(p); break;
    case MXQ_DTYPE_F32 * 2 + 1: w4a8_g128_kernel<0, true, kBM><<<grid, kThreads, 0, st>>>(p); break;
    case MXQ_DTYPE_F16 * 2: w4a8_g128_kernel<1, false, kBM><<<grid, kThreads, 0, st>>>(p); break;
    case MXQ_DTYPE_F16 * 2 + 1: w4a8_g128_kernel<1, true, kBM><<<grid, kThreads, 0, st>>>(p); break;
    case MXQ_DTYPE_BF16 * 2: w4a8_g128_kernel<2, false, kBM><<<grid, kThreads, 0, st>>>(p); break;
    case MXQ_DTYPE_BF16 * 2 + 1: w4a8_g128_kernel<2, true, kBM><<<grid, kThreads, 0, st>>>(p); break;
    default: return mxq_set_error(MXQ_ERR_UNSUPPORTED, "output dtype code %d", out_dtype);
  }
  return mxq_check_launch("w4a8_g128_kernel");
}

}  // namespace

int launch_w4_g128(W4Args p, int out_dtype, bool prepared, hipStream_t st) {
  if (p.M * p.K >= (int64_t)1 << 31 || p.N * (p.K / 2) >= (int64_t)1 << 31 || p.N * (p.K / 128) * 2 >= (int64_t)1 << 31)
    return MXQ_ERR_UNSUPPORTED;  // the caller falls back to the general kernel
  // 128-row tiles unless they would leave CUs with fewer than two workgroups (256 CUs).
  const int64_t tiles128 = ((p.M + 127) / 128) * ((p.N + kBN - 1) / kBN);
  return tiles128 >= 2 * 256 ? launch_tiles<128>(p, out_dtype, prepared, st)
                             : launch_tiles<64>(p, out_dtype, prepared, st);
}

}  // namespace mxq
