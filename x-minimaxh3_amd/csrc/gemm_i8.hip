// INT8 x INT8 -> INT32 GEMM on gfx950 matrix cores, with fused epilogues.
//
// C[m, n] = sum_k A[m, k] * B[n, k]: A [M, K] activations, B [N, K] weights, both K-contiguous
// (the reference's torch._int_mm(x_8, weight.T) / CUTLASS RowMajor x ColumnMajor,
// backends/turbo/vendor/comfy_kitchen/backends/cuda/ops/cutlass_gemm_int8.cu:245-283).
//
// Main loop: one workgroup per CU owns a 256 x 256 output tile. K advances 128 bytes per stage; a
// stage's A and B chunks (32 KB each) are fetched with gfx950's direct-to-LDS 16-byte loads into
// a ring of five 32 KB slots, one to two stages ahead of the MFMAs, so global latency hides behind
// matrix work and no VGPRs stage data. Fragment reads are inline-asm ds_read_b128 with explicit
// lgkmcnt waits; vmcnt waits and barriers are issued by hand too (s_waitcnt + s_barrier) so that
// the prefetches stay in flight across the barrier that publishes the next stage.
//  * Ping-pong (the plain epilogues): 512 threads, two waves per SIMD, each owning 128 x 64 as a
//    4 x 2 grid of v_mfma_i32_32x32x32_i8 blocks (128 int32 accumulators per lane). The SIMD's
//    two waves take turns: one issues a half stage of MFMAs while the other reads its next
//    fragments and issues operand loads, a barrier between turns (pp_main_loop).
//  * Four waves (the table epilogues, whose 128 KB table leaves no LDS for eight waves' output
//    staging): 256 threads, one wave per SIMD owning 128 x 128 as 4 x 4 blocks (256 accumulators
//    per lane, in AGPRs), each K-step's fragment reads issued behind the previous step's MFMAs and
//    the operand loads interleaved one per MFMA.
// Problems with fewer 256-tiles than CUs run the four-wave code on 128 x 128 tiles: two
// workgroups per CU, or, when all the 128-tiles fit on the CUs at once, one per CU with a
// nine-slot ring four stages deep -- as 128 x 96 tiles (four 32-row wave strips) when those
// still fit and are more numerous, so that more CUs share the work.
//
// Epilogue: the MFMAs run with the weights as first operand, so each lane's accumulators are
// one output row in four runs of four consecutive columns. Every output type is converted in
// registers and stored as 8- or 16-byte runs (lanes l and l + 32 cover adjacent runs); the
// per-row scale is one register per 32-row block and row reductions stay inside lane pairs.
//   kEpiI32     raw int32 accumulators.
//   kEpiDequant y = out(fp32(acc) * (xs[m] * ws[n])); y = out(y + bias[n])
//               (backends/eager/quantization.py:1031-1054; single IEEE ops, -ffp-contract=off).
//   kEpiGelu    bf16 dequant as above, then h = gelu_tanh(y) in bf16 (table in LDS), and the
//               per-row absmax of h folded into row_absmax[m] with atomics (it feeds the next
//               layer's quantizer, backends/_activations.py:40-53 + quantization.py:857-875).
//   kEpiSwiGLU  bf16 dequant as above of a SwiGLU fc1 whose weight rows come in blocks of 16 gate
//               rows then the 16 matching up rows (prepare_swiglu_fc1 on the host), then
//               h = bf16(bf16(silu(gate)) * up) (table in LDS) written as [M, N/2]: the fused
//               form of int8_linear followed by fc2's input_act="swiglu"
//               (CK/backends/_activations.py:50-52, h3serve/native_engine/model/fused_mlp.py:386-420).
//   kEpiGatedRes bf16 dequant as above, then the gated residual update in place:
//               res[m, n] = bf16(res[m, n] + y * gate[gate_rows[m], n])  (the reference's
//               addcmul_ after fc2, h3serve/native_engine/model/layers.py:944-960 and
//               fused_mlp.py:157-219; y * gate is exact in fp32, so one fp32 add, then RNE).

#include "act_rot.h"

namespace mxq {

constexpr int kBK = 128;                                // K bytes per stage
constexpr int kGemmThreads = 256;                       // 4 waves as 2 x 2

// Tile shapes: kT x kT outputs per workgroup, each wave (kT/2)^2 as kBI x kBJ MFMA blocks of
// 32 x 32. 256: one workgroup per CU, 160 KB ring, the GEMM of large problems. 128: two
// workgroups per CU, 80 KB ring, for problems with fewer 256-tiles than CUs. 128 with kDeep:
// one workgroup per CU with a 144 KB ring that holds four stages in flight instead of two, for
// problems whose 128-tiles all fit on the CUs at once (one workgroup per CU then leaves the
// main loop waiting on operand latency, not on other workgroups).
// kTN = 96 (deep ring only): 128 x 96 tiles, the four waves stacked as 32-row strips of 1 x 3
// blocks, for problems that fill more CUs that way (1024 x 3072: 256 tiles instead of 192 of 128).
// A B chunk is then 12 KB in a 16 KB slot, and the ring carries 28 KB per stage instead of 32.
template <int kT, bool kDeep = false, bool kPP = false, int kTN = kT>
struct TileCfg {
  static_assert(kT == 128 || !kDeep, "the deep ring exists for 128-tiles only");
  static_assert(kT == 256 || !kPP, "the ping-pong schedule exists for 256-tiles only");
  static_assert(kTN == kT || (kDeep && kTN == 96), "128 x 96 tiles run the deep ring only");
  static constexpr bool kPingPong = kPP;
  static constexpr int kWaves = kPP ? 8 : 4;                    // two per SIMD with kPP
  static constexpr int kThreads = kWaves * 64;
  static constexpr int kBM = kT, kBN = kTN;
  static constexpr int kWavesN = kPP ? 4 : (kTN == kT ? 2 : 1);  // waves across the tile's columns
  static constexpr int kWaveM = kPP ? kT / 2 : kT / (kWaves / kWavesN), kWaveN = kTN / kWavesN;
  static constexpr int kBI = kWaveM / 32, kBJ = kWaveN / 32;
  static constexpr int kSlotBytes = kT * kBK;                  // one operand chunk of a stage (slot size)
  static constexpr int kLoads = kSlotBytes / 1024 / kWaves;     // direct-to-LDS loads per wave per A slot
  static constexpr int kLoadsB = kTN * kBK / 1024 / kWaves;     // ... per B slot
  static constexpr int kAhead = kDeep ? 4 : 2;                  // stages requested ahead of the MFMAs
  static constexpr int kSlots = 2 * kAhead + 1;                 // LDS ring of operand chunks
  static constexpr int kLds = kSlots * kSlotBytes;
  static constexpr int kEpiLds = kT == 256 ? 131072 : 4 * kSlotBytes;  // per-column factors
  static constexpr int kPerCu = kT == 256 || kDeep ? 1 : 2;     // workgroups per CU
  static_assert(kLds <= 160 * 1024, "the ring exceeds the CU's LDS");
  static_assert(kAhead * (kLoads + kLoadsB) < 64, "loads in flight exceed the vmcnt counter");
  static_assert(kWaveM % 32 == 0 && kWaveN % 32 == 0 && kTN % (8 * kWaves) == 0, "tile split");
};
// Tile-rows per group for problems of several rounds: with 2, the ~32 tiles an XCD runs at once are
// 2 tile-rows x 16 tile-columns, so an activation panel is read from HBM once and then served
// from that XCD's L2 to the whole row sweep, and the weight panels (the smaller operand) come
// back from the last-level cache. For the four-wave kernels, measured against 1, 3, 4, 8, 16 and
// 32 on the FFN and QKV shapes at 720p, 2 was fastest (fc1 -2.8 %, fc2 -3.2 %, QKV -2 % against
// 8). The ping-pong kernel (a third more LDS traffic per MFMA, so a lower clock under the board's
// power limit) does better with the fewer L2 fills of 4-row groups (QKV -1 to -2 %, FFN -0.3 %
// against 2; 1, 6 and 8 slower), also as looping workgroups (against 4: 3 the same on the FFN
// chain and 0.4 % slower on QKV, 5 +0.7 %, 6 +1.3 %, 8 +3 %). Problems of one round choose their
// own (plan_gemm).
constexpr int kGroupM = 2, kGroupMPingPong = 4;

enum { kEpiI32 = 0, kEpiDequant = 1, kEpiGelu = 2, kEpiGatedRes = 3, kEpiSwiGLU = 4 };
// Table epilogues as plan_gemm sees them: GELU keeps the whole 128 KB table in LDS (four-wave
// 256-tiles), SwiGLU the 8 KB compact SiLU table (ping-pong 256-tiles).
enum { kTableGelu = 1, kTableSwiGLU = 2 };

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
  int vec_store;   // run stores allowed (d aligned to 4 elements and ldd % 4 == 0)
  int line_store;  // 16-byte row pieces allowed (every row of d, and of res / gate, 16-byte aligned)
  int tiles_m, tiles_n;
  // kEpiGatedRes: bf16 residual [M, ldr] (read and written), bf16 gate [*, ldg], gate_rows [M]
  uint16_t* res;
  const uint16_t* gate;
  const int32_t* gate_rows;
  int64_t ldr, ldg, gate_count;
  // Balanced tile queue: the last `pool` tiles of each XCD's range are claimed at run time, by
  // that XCD's workgroups first and then by any XCD's (see pick_tile). grid = 8 * wg_per_xcd;
  // n_claim workgroups claim; counters (the caller's workspace) hold the claim counts.
  int pool, wg_per_xcd, n_claim;
  unsigned* counters;
  int group_m;  // tile-rows per group of the tile order (tile_walk)
  // Ping-pong kernel only: wg_per_xcd workgroups per XCD loop over the tiles, claiming them from
  // the counters (pp_tiles); n_claim is then the grid.
  int persistent;
};

// LDS operand layout: a tile row is 128 bytes = eight 16-byte chunks; chunk c of row r sits at
// slot c ^ f(r), f(r) = (r >> 1) & 7. gfx950 serves a ds_read_b128 sixteen lanes per clock:
// an MFMA operand read has those lanes on sixteen consecutive rows at one chunk, and the map
// gives them sixteen distinct (r & 1, slot) pairs, i.e. all 64 banks once.
MXQ_DEVICE int swz_f(int r) { return (r >> 1) & 7; }
MXQ_DEVICE int swz(int r, int c) { return r * kBK + ((c ^ swz_f(r)) << 4); }

// threadIdx.x read through an empty asm statement: what is computed from it cannot be hoisted
// out of the ping-pong kernel's tile loop (lane addresses kept live across the main loop spilled).
MXQ_DEVICE int tid_x() {
  int t = threadIdx.x;
  __asm__ volatile("" : "+v"(t));
  return t;
}

// Zero source for the K tail of A (B's tail may hold anything: it meets zeros).
static __device__ __attribute__((aligned(16))) uint8_t kZeroChunk[16];

// Tile order: first spread contiguous tile ranges over the 8 XCDs (workgroup ids are dealt to
// XCDs round-robin), then walk each range in groups of group_m tile-rows so that the tiles
// resident on one XCD share A and B panels in that XCD's L2. tile_walk maps a position t of
// that order to its tile row and column.
MXQ_DEVICE void tile_walk(int t, int tiles_m, int tiles_n, int group_m, int& tm, int& tn) {
  const int group = group_m * tiles_n;
  const int g = t / group;
  const int first_m = g * group_m;
  const int gm = min(tiles_m - first_m, group_m);
  const int in = t % group;
  tm = first_m + in % gm;
  tn = in / gm;
}

// Static order: workgroup bid takes position (bid % 8) * per + bid / 8, i.e. XCD x runs
// positions [x * per, (x + 1) * per); the last num % 8 positions are taken in id order.
MXQ_DEVICE int static_position(int bid, int num) {
  const int per = num / 8;
  return bid < per * 8 ? (bid % 8) * per + bid / 8 : bid;
}

// XCD x's range of positions in the balanced order: [start, start + count), the num % 8
// leftover positions going one each to the first XCDs.
MXQ_DEVICE void xcd_range(int x, int num, int& start, int& count) {
  const int per = num / 8, rem = num % 8;
  start = x * per + min(x, rem);
  count = per + (x < rem ? 1 : 0);
}

// Direct-to-LDS stage loads (global_load_lds_dwordx4). One instruction fills 1 KB of LDS:
// lane i writes slot i % 8 of tile row 8 b + i / 8, so the lane fetches logical chunk
// (i % 8) ^ f(row) of that row, and eight lanes read one whole 128-byte line of the row-major
// operand (half lines, as 64-byte steps would read, halve the L2 -> CU throughput). Wave w
// loads blocks b = kL w .. kL w + kL - 1 of each A and B slot.
template <int kL, int kLB = kL>
struct Loader {
  const int8_t* a[kL];
  const int8_t* b[kLB];
  int koff[2];   // logical chunk offset (bytes) of this lane's piece in 8-row block 2i and 2i + 1
  int wave;      // the wave's index, as a scalar: LDS destinations (M0) are then scalar arithmetic
};

// A load's 8-row block b = wave * (loads per slot) + t: the chunk swizzle of its rows depends on
// b only through b & 1 (swz_f(8 b + l / 8) = 4 (b & 1) + l / 16).
template <int kL>
MXQ_DEVICE int load_parity(int wave, int t) { return (wave * kL + t) & 1; }

template <int kL, int kLB>
MXQ_DEVICE void make_loader(Loader<kL, kLB>& L, const GemmArgs& p, int64_t m0, int64_t n0) {
  const int w = tid_x() >> 6, lane = tid_x() & 63;
  L.wave = __builtin_amdgcn_readfirstlane(w);
  // (the operand bases pass an empty asm statement too, so that their register copies are not
  // hoisted out of the ping-pong kernel's tile loop either)
  const int8_t* a = p.a;
  const int8_t* b = p.b;
  __asm__ volatile("" : "+s"(a), "+s"(b));
#pragma unroll
  for (int par = 0; par < 2; ++par) L.koff[par] = ((lane & 7) ^ swz_f(par * 8 + (lane >> 3))) * 16;
#pragma unroll
  for (int t = 0; t < kL; ++t) {
    const int r = (w * kL + t) * 8 + (lane >> 3);
    L.a[t] = a + min(m0 + r, p.M - 1) * p.K + ((lane & 7) ^ swz_f(r)) * 16;
  }
#pragma unroll
  for (int t = 0; t < kLB; ++t) {
    const int r = (w * kLB + t) * 8 + (lane >> 3);
    L.b[t] = b + min(n0 + r, p.N - 1) * p.K;
  }
}

// Load t of this wave's share of an A (kB = false) or B slot. With kCheck a chunk past K reads
// zeros (A) or any valid bytes (B: their products with A's zeros vanish); without it the caller
// guarantees the whole stage lies below K.
template <bool kB, bool kCheck, int kL, int kLB>
MXQ_DEVICE void issue_one(const Loader<kL, kLB>& L, char* slot, int64_t k0, int64_t K, int t) {
  constexpr int kN = kB ? kLB : kL;
  const int w = L.wave;
  // (a select, not an index: a run-time index would put the pair in scratch memory)
  const int koff = load_parity<kN>(w, t) ? L.koff[1] : L.koff[0];
  const void* src;
  if constexpr (kCheck) {
    const bool kin = k0 + koff < K;
    src = kB ? (kin ? (const void*)(L.b[t] + k0 + koff) : (const void*)L.b[t])
             : (kin ? (const void*)(L.a[t] + k0) : (const void*)kZeroChunk);
  } else {
    src = kB ? (const void*)(L.b[t] + k0 + koff) : (const void*)(L.a[t] + k0);
  }
  __builtin_amdgcn_global_load_lds((gptr_t)src, (lptr_t)(slot + (w * kN + t) * 1024), 16, 0, 0);
}

template <bool kB, int kL, int kLB>
MXQ_DEVICE void issue_slot(const Loader<kL, kLB>& L, char* slot, int64_t k0, int64_t K) {
#pragma unroll
  for (int t = 0; t < (kB ? kLB : kL); ++t) issue_one<kB, true>(L, slot, k0, K, t);
}

// Fragments of K-step ks (32 K-bytes) of a stage: A rows wrow + i*32 + l%32 and B rows
// wcol + j*32 + l%32 (the wave's first row and column in the tile, multiples of 16), chunk
// ks*2 + l/32. Every row a lane touches has the same swizzle f = ((l % 32) >> 1) & 7, so one base
// address per operand serves all its blocks.
template <class C>
MXQ_DEVICE void load_frags(int lane, uint32_t slot_a, uint32_t slot_b, int wrow, int wcol, int ks, v4i fa[C::kBI],
                           v4i fb[C::kBJ]) {
  const int lr = lane & 31;
  const uint32_t x = (uint32_t)(((ks * 2 + (lane >> 5)) ^ swz_f(lr)) << 4);
  const uint32_t ba = slot_a + (uint32_t)(wrow + lr) * kBK + x;
  const uint32_t bb = slot_b + (uint32_t)(wcol + lr) * kBK + x;
  static_for<C::kBI>([&](auto I) { fa[decltype(I)::value] = lds_read_b128<decltype(I)::value * 32 * kBK>(ba); });
  static_for<C::kBJ>([&](auto J) { fb[decltype(J)::value] = lds_read_b128<decltype(J)::value * 32 * kBK>(bb); });
}

// The MFMAs compute C^T blocks (weights as the first operand): lane l of a 32 x 32 block then
// holds output row l % 32 and, in registers r = 0..15, output columns
// (r / 4) * 8 + (l / 32) * 4 + r % 4 -- four runs of four consecutive columns of one row.
template <class C>
MXQ_DEVICE void mma_step(const v4i fa[C::kBI], const v4i fb[C::kBJ], v16i acc[C::kBI][C::kBJ]) {
#pragma unroll
  for (int i = 0; i < C::kBI; ++i)
#pragma unroll
    for (int j = 0; j < C::kBJ; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fb[j], fa[i], acc[i][j], 0, 0, 0);
}

// The MFMAs of one K-step with kCount direct-to-LDS loads (loads kFirst .. of one operand slot)
// interleaved, one after each of the first kCount MFMAs (kCount <= kBI * kBJ). Spread this way,
// a load that waits for room in the memory pipeline holds up the wave while its MFMAs still
// run, rather than after the last of them.
template <class C, bool kB, int kFirst, int kCount, bool kCheck>
MXQ_DEVICE void mma_step_dma(const v4i fa[C::kBI], const v4i fb[C::kBJ], v16i acc[C::kBI][C::kBJ],
                             const Loader<C::kLoads, C::kLoadsB>& L, char* slot, int64_t k0, int64_t K, bool on) {
  static_assert(kCount <= C::kBI * C::kBJ, "more loads than MFMAs to spread them over");
#pragma unroll
  for (int q = 0; q < C::kBI * C::kBJ; ++q) {
    const int i = q / C::kBJ, j = q % C::kBJ;
    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fb[j], fa[i], acc[i][j], 0, 0, 0);
    if (q < kCount && on) issue_one<kB, kCheck>(L, slot, k0, K, kFirst + q);  // t is a constant once unrolled
  }
}

// One run of four consecutive outputs as store words: fp32/int32 outputs give four words,
// 16-bit outputs two words of two values each (the lower column in the low half).
// Dequant: y = out(fp32(acc) * (xs * ws)); y = out(y + bias). A missing bias is passed as
// -0.0, for which y + (-0.0) == y for every y (signed zeros, infinities and NaN included).
template <int kEpi, int kOut>
MXQ_DEVICE void epi_run(const v16i& acc, int q, float xs, const float* w, const float* bias,
                        uint32_t* out) {
  if constexpr (kEpi == kEpiI32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = (uint32_t)acc[q * 4 + e];
  } else if constexpr (kOut == 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float y = (float)acc[q * 4 + e] * (xs * w[e]);
      out[e] = __float_as_uint(y + bias[e]);
    }
  } else if constexpr (kOut == 1) {
    uint32_t h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float y = round_f16((float)acc[q * 4 + e] * (xs * w[e]));
      h[e] = f32_to_f16_bits(y + bias[e]);
    }
    out[0] = h[0] | (h[1] << 16);
    out[1] = h[2] | (h[3] << 16);
  } else {
    float y[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = round_bf16((float)acc[q * 4 + e] * (xs * w[e])) + bias[e];
    out[0] = pack_bf16x2(y[0], y[1]);
    out[1] = pack_bf16x2(y[2], y[3]);
  }
}

// Store one run (words as produced by epi_run) of row `row` from column `col`. `fast`: the
// caller has established that the four columns are inside the output and the run aligned.
// The epilogue's vector stores are nontemporal: the output is not read again by this launch,
// and keeping it out of the L2 leaves that to the operand panels the tiles share (FFN chain at
// 720p: fc1 6.54 -> 6.46 ms, the chain 13.45 -> 13.35 ms on one box).
template <int kElem>
MXQ_DEVICE void store_run(void* d, int64_t ldd, int64_t row, int64_t col, int64_t N, bool fast,
                          const uint32_t* w) {
  char* base = reinterpret_cast<char*>(d) + (row * ldd + col) * kElem;
  if (fast) {
    if constexpr (kElem == 4)
      __builtin_nontemporal_store(v4u{w[0], w[1], w[2], w[3]}, reinterpret_cast<v4u*>(base));
    else
      __builtin_nontemporal_store(v2u{w[0], w[1]}, reinterpret_cast<v2u*>(base));
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (col + e < N) {
        if constexpr (kElem == 4)
          reinterpret_cast<uint32_t*>(base)[e] = w[e];
        else
          reinterpret_cast<uint16_t*>(base)[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
      }
    }
  }
}

// Stores the four runs of one 32 x 32 block row. Interior tiles (`full`) store unguarded.
template <int kElem>
MXQ_DEVICE void store_block_row(const GemmArgs& p, bool full, int64_t row, int64_t col0,
                                const uint32_t* w) {
  constexpr int kWords = kElem == 4 ? 4 : 2;
  if (full) {
#pragma unroll
    for (int q = 0; q < 4; ++q) store_run<kElem>(p.d, p.ldd, row, col0 + q * 8, p.N, true, w + q * kWords);
  } else if (row < p.M) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t col = col0 + q * 8;
      store_run<kElem>(p.d, p.ldd, row, col, p.N, p.vec_store && col + 4 <= p.N, w + q * kWords);
    }
  }
}

// Gated residual update of one 32 x 32 block row (four runs of four columns, bf16 words as
// produced by epi_run): res = bf16(res + y * gate[grow]). Interior tiles (`full`, with the
// residual and gate rows 8-byte aligned) use 8-byte accesses.
MXQ_DEVICE uint32_t gated_pair(uint32_t r, uint32_t y, uint32_t g) {
  const float lo = bf16_to_f32(r & 0xFFFFu) + bf16_to_f32(y & 0xFFFFu) * bf16_to_f32(g & 0xFFFFu);
  const float hi = bf16_to_f32(r >> 16) + bf16_to_f32(y >> 16) * bf16_to_f32(g >> 16);
  return pack_bf16x2(lo, hi);
}

MXQ_DEVICE void gated_block_row(const GemmArgs& p, bool full, int64_t row, int64_t grow, int64_t col0,
                                const uint32_t* w) {
  uint16_t* __restrict__ res = p.res;
  const uint16_t* __restrict__ gate = p.gate;
  if (full) {
    v2u r[4], g[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      r[q] = *reinterpret_cast<const v2u*>(res + row * p.ldr + col0 + q * 8);
      g[q] = *reinterpret_cast<const v2u*>(gate + grow * p.ldg + col0 + q * 8);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<v2u*>(res + row * p.ldr + col0 + q * 8) =
          v2u{gated_pair(r[q][0], w[2 * q], g[q][0]), gated_pair(r[q][1], w[2 * q + 1], g[q][1])};
  } else if (row < p.M) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t col = col0 + q * 8 + e;
        if (col < p.N) {
          const uint32_t y = (w[2 * q + (e >> 1)] >> (16 * (e & 1))) & 0xFFFFu;
          const float v = bf16_to_f32(res[row * p.ldr + col]) + bf16_to_f32(y) * bf16_to_f32(gate[grow * p.ldg + col]);
          res[row * p.ldr + col] = (uint16_t)f32_to_bf16_bits(v);
        }
      }
    }
  }
}

// ---- whole-line stores through LDS ----
// Stored straight from the accumulator layout, every store instruction writes 8- or 16-byte
// pieces of 32 different rows. Interior tiles instead pass 32-row x 128-byte pieces of a wave's
// output through a private 4 KB LDS buffer: written in the accumulator layout, read back by rows
// (read t gives lane l 16 bytes of row 8 t + l / 8), so that eight lanes store one whole
// 128-byte line. Chunk c (16 bytes) of row r sits at chunk c ^ ((r >> 1) & 7) of the row: the
// writes (32 rows at one chunk) and the reads (8 rows x 8 chunks) then use every bank equally.
constexpr int kStageBytes = 32 * 128;

MXQ_DEVICE char* stage_at(char* buf, int r, int c) { return buf + r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }

// Lanes exchange data through the buffer: this orders the wave's LDS accesses before the call
// against those after it (one wave's LDS instructions execute in order).
MXQ_DEVICE void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The 8 bytes of half h of chunk c of row r.
// The staging accesses are inline assembly (lds_write_*, lds_read_b128): the ping-pong kernel
// runs its epilogue while the next tile's first operand loads land in other LDS slots.
MXQ_DEVICE void stage_put8(char* buf, int r, int c, int h, uint32_t w0, uint32_t w1) {
  lds_write_b64(lds_addr(stage_at(buf, r, c) + h * 8), v2u{w0, w1});
}

MXQ_DEVICE void stage_put16(char* buf, int r, int c, const uint32_t* w) {
  lds_write_b128(lds_addr(stage_at(buf, r, c)), v4u{w[0], w[1], w[2], w[3]});
}

// Row-order reads t = 0..3 of the staged piece; the caller waits for them (stage_wait).
MXQ_DEVICE void stage_get4(char* buf, v4u (&v)[4]) {
  const int lane = tid_x() & 63;
#pragma unroll
  for (int t = 0; t < 4; ++t)
    v[t] = __builtin_bit_cast(v4u, lds_read_b128<0>(lds_addr(stage_at(buf, t * 8 + (lane >> 3), lane & 7))));
}

MXQ_DEVICE void stage_wait() {
  wait_lgkm<0>();
  __builtin_amdgcn_sched_barrier(0);
}

// Stores the staged piece as bytes [byte0, byte0 + 128) of rows row0 .. row0 + 31 of d.
MXQ_DEVICE void stage_store(const GemmArgs& p, char* buf, int64_t row0, int64_t byte0, int64_t pitch) {
  const int lane = tid_x() & 63;
  wave_lds_sync();
  v4u v[4];
  stage_get4(buf, v);
  stage_wait();
  char* base = reinterpret_cast<char*>(p.d) + (row0 + (lane >> 3)) * pitch + byte0 + (lane & 7) * 16;
#pragma unroll
  for (int t = 0; t < 4; ++t) __builtin_nontemporal_store(v[t], reinterpret_cast<v4u*>(base + t * 8 * pitch));
}

// The same for a piece of 64 bytes per row (chunks 0-3): rows row0 .. row0 + 31 of d, bytes
// [byte0, byte0 + 64), two 16-byte stores per lane. (Pairing two ping-pong waves' halves into
// whole lines behind a workgroup barrier measured 0.7 % slower on the SwiGLU fc1.)
MXQ_DEVICE void stage_store64(const GemmArgs& p, char* buf, int64_t row0, int64_t byte0, int64_t pitch) {
  const int lane = tid_x() & 63;
  wave_lds_sync();
  v4u v[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
    v[t] = __builtin_bit_cast(v4u, lds_read_b128<0>(lds_addr(stage_at(buf, t * 16 + (lane >> 2), lane & 3))));
  stage_wait();
  char* base = reinterpret_cast<char*>(p.d) + (row0 + (lane >> 2)) * pitch + byte0 + (lane & 3) * 16;
#pragma unroll
  for (int t = 0; t < 2; ++t) __builtin_nontemporal_store(v[t], reinterpret_cast<v4u*>(base + t * 16 * pitch));
}

// Two 32 x 32 blocks of 16-bit words (jj = 0, 1: 8 words each, as epi_run gives them), or one
// block of 32-bit words, as one piece.
MXQ_DEVICE void stage_blocks16(char* buf, const uint32_t (&w)[2][8]) {
  const int lane = tid_x() & 63;
  wave_lds_sync();  // the previous piece has been read
#pragma unroll
  for (int jj = 0; jj < 2; ++jj)
#pragma unroll
    for (int q = 0; q < 4; ++q) stage_put8(buf, lane & 31, jj * 4 + q, lane >> 5, w[jj][2 * q], w[jj][2 * q + 1]);
}

MXQ_DEVICE void stage_block32(char* buf, const uint32_t* w) {
  const int lane = tid_x() & 63;
  wave_lds_sync();
#pragma unroll
  for (int q = 0; q < 4; ++q) stage_put16(buf, lane & 31, q * 2 + (lane >> 5), w + q * 4);
}

// Gated residual update of a staged piece (bf16 y of rows row0 .. row0 + 31, columns
// col0 .. col0 + 63): res = bf16(res + y * gate[grow]) with 16-byte accesses; grow[t] is the
// gate row of row row0 + 8 t + lane / 8. The residual and gate reads are issued before the
// staging so that their latency overlaps it.
MXQ_DEVICE void gated_lines(const GemmArgs& p, char* buf, int64_t row0, int64_t col0, const int64_t (&grow)[4],
                            const uint32_t (&w)[2][8]) {
  const int lane = tid_x() & 63;
  uint16_t* res = p.res + (row0 + (lane >> 3)) * p.ldr + col0 + (lane & 7) * 8;
  v4u r[4], g[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    r[t] = *reinterpret_cast<const v4u*>(res + t * 8 * p.ldr);
    g[t] = *reinterpret_cast<const v4u*>(p.gate + grow[t] * p.ldg + col0 + (lane & 7) * 8);
  }
  stage_blocks16(buf, w);
  wave_lds_sync();
  v4u ys[4];
  stage_get4(buf, ys);
  stage_wait();
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const v4u y = ys[t];
    __builtin_nontemporal_store(
        v4u{gated_pair(r[t][0], y[0], g[t][0]), gated_pair(r[t][1], y[1], g[t][1]),
            gated_pair(r[t][2], y[2], g[t][2]), gated_pair(r[t][3], y[3], g[t][3])},
        reinterpret_cast<v4u*>(res + t * 8 * p.ldr));
  }
}

// ---- balanced tile queue ----
// The hardware deals workgroup ids to the 8 XCDs round-robin, so with a static order each XCD
// runs exactly 1/8 of the tiles, and the XCDs do not run at one speed: per-workgroup timestamps
// of a 75600 x 5120 x 20480 GEMM gave mean tile times from 282 to 303 us by XCD, and the last
// XCD finished 0.5 ms after the first. Here workgroup (x = bid % 8, k = bid / 8) takes position
// start_x + k of its XCD's range while k < count_x - pool; the rest of the range (the pool) and
// a few extra workgroups per XCD claim positions at run time: first from their own XCD's pool,
// then from the other pools in turn. A fast XCD thus takes over the end of a slow one's range;
// workgroups that find every pool empty exit. Claims are relaxed agent-scope atomics on the
// pool counters (no data passes between workgroups); each claiming workgroup then counts itself
// with an acquire-release increment, and the one that makes the count complete resets the
// counters for the next launch, after every claim of this one. Thread 0 claims, the
// workgroup reads the result through lds[0] before the ring is used. Returns the position, or
// -1 if the workgroup has nothing to do.
MXQ_DEVICE int pick_tile(const GemmArgs& p, int num, char* lds) {
  const int bid = blockIdx.x;
  if (p.pool == 0) return static_position(bid, num);
  const int x = bid & 7, k = bid >> 3;
  int start, count;
  xcd_range(x, num, start, count);
  if (k < count - p.pool) return start + k;
  volatile int* shared_pos = reinterpret_cast<volatile int*>(lds);
  if (threadIdx.x == 0) {
    int got = -1;
    for (int j = 0; j < 8 && got < 0; ++j) {
      const int y = (x + j) & 7;
      const unsigned i = __hip_atomic_fetch_add(p.counters + y * 32, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (i < (unsigned)p.pool) {
        int ys, yc;
        xcd_range(y, num, ys, yc);
        got = ys + yc - p.pool + (int)i;
      }
    }
    // Release: this workgroup's claims above are ordered before its count; acquire: the last
    // claimer sees every claim of the launch (the counts form one release sequence) before it
    // resets the pools, so no claim can land on a counter after its reset.
    const unsigned done = __hip_atomic_fetch_add(p.counters + 8 * 32, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (done == (unsigned)p.n_claim - 1) {  // every claim of this launch has been made
      for (int y = 0; y < 8; ++y) __hip_atomic_exchange(p.counters + y * 32, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_exchange(p.counters + 8 * 32, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    *shared_pos = got;
  }
  __syncthreads();
  const int pos = *shared_pos;
  __syncthreads();  // read before the ring's first loads overwrite lds[0]
  return pos;
}

// ---- ping-pong main loop (kPP: eight waves, two per SIMD) ----
// Waves w and w + 4 share a SIMD and a 128 x 128 quadrant of the 256 x 256 tile, one 64-column
// half each (128 accumulators per lane, so two waves fit a SIMD's registers). They alternate: in
// every phase one group of four waves (one per SIMD) issues the 16 MFMAs of a half stage (two
// K-steps) from fragments already in registers, while the other group reads its fragments of the
// next half stage from LDS and issues its share of the direct-to-LDS operand loads; a workgroup
// barrier ends each phase. A wave's stalls on LDS latency, load issue or the barrier thus fall in
// the phases where the other wave of its SIMD keeps the matrix pipe busy.
//
// Ring: the operand chunks A_0 B_0 A_1 B_1 ... go to slot (chunk index) % 5 as in the four-wave
// loop. Iteration kt (stage kt in slots sa, sb) has four phases; group g computes in phases
// 2q + g and reads in the others:
//   P0  g0: MFMAs of (kt, K-steps 0-1)     g1: reads (kt, 0-1), loads A_kt+2 into B_kt-1's slot
//   P1  g1: MFMAs of (kt, 0-1)             g0: reads (kt, 2-3), loads A_kt+2
//   P2  g0: MFMAs of (kt, 2-3)             g1: reads (kt, 2-3)        both then wait for stage kt+1
//   P3  g1: MFMAs of (kt, 2-3) + loads     g0: reads (kt+1, 0-1), loads B_kt+2 into A_kt's slot
//       of B_kt+2 into A_kt's slot
// A_kt+2's slot was last read in P2 of iteration kt-1 and A_kt's in P2 of this one, so every
// load goes to a slot no wave reads any more; stage kt+1 is complete (each wave waited for its
// own loads of it, vmcnt) before the barrier that opens P3, its first reader.
template <class C>
MXQ_DEVICE void pp_frags(int lane, uint32_t slot_a, uint32_t slot_b, int wrow, int wcol, int ks0, v4i (&fa)[2][C::kBI],
                         v4i (&fb)[2][C::kBJ]) {
  load_frags<C>(lane, slot_a, slot_b, wrow, wcol, ks0, fa[0], fb[0]);
  load_frags<C>(lane, slot_a, slot_b, wrow, wcol, ks0 + 1, fa[1], fb[1]);
}

// The 16 MFMAs of a half stage; with kLoadsB > 0 one direct-to-LDS load (t = 0 .. kLoadsB-1 of a
// B slot) follows each of the first kLoadsB MFMAs when `on`.
template <class C, int kLoadsB, bool kCheck>
MXQ_DEVICE void pp_mma(const v4i (&fa)[2][C::kBI], const v4i (&fb)[2][C::kBJ], v16i (&acc)[C::kBI][C::kBJ],
                       const Loader<C::kLoads>& L, char* slot, int64_t k0, int64_t K, bool on) {
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int q = 0; q < C::kBI * C::kBJ; ++q) {
      const int i = q / C::kBJ, j = q % C::kBJ;
      acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fb[kk][j], fa[kk][i], acc[i][j], 0, 0, 0);
      if (kk == 0 && q < kLoadsB && on) issue_one<true, kCheck>(L, slot, k0, K, q);
    }
}

template <bool kB, bool kCheck, int kL>
MXQ_DEVICE void pp_issue(const Loader<kL>& L, char* slot, int64_t k0, int64_t K, bool on) {
  if (on) {
#pragma unroll
    for (int t = 0; t < kL; ++t) issue_one<kB, kCheck>(L, slot, k0, K, t);
  }
}

MXQ_DEVICE void pp_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  barrier_no_drain();
  __builtin_amdgcn_sched_barrier(0);
}

// One group's whole main loop (kG = 0: waves 0-3, 1: waves 4-7). The two groups run separate
// straight-line code with the same barriers, so no accumulator or fragment value depends on a
// branch (a branch per phase made the compiler copy and spill them).
// `before_tail` runs ahead of the last two or three iterations (the epilogue's factor reads, whose
// latency then hides behind those iterations' MFMAs).
template <class C, int kG, class BeforeTail>
MXQ_DEVICE void pp_loop(const GemmArgs& p, char* lds, v16i (&acc)[C::kBI][C::kBJ], int wrow, int wcol,
                        const Loader<C::kLoads>& ld, BeforeTail&& before_tail) {
  constexpr int kSlotBytes = C::kSlotBytes, kSlots = C::kSlots, kL = C::kLoads;
  const int ktiles = (int)((p.K + kBK - 1) / kBK);
  const uint32_t lds_addr = (uint32_t)(uintptr_t)(lptr_t)lds;
  auto slot_addr = [&](int sl) { return lds_addr + (uint32_t)(sl * kSlotBytes); };
  const int lane = tid_x() & 63;  // (once per tile: what the fragment reads derive from it stays out of the K loop)

  // prologue: A_0, B_0 and A_1 were issued into slots 0-2 before (pp_first_loads); B_1 goes to
  // slot 3 once every wave is done with the previous tile's epilogue (factors in slot 3, staging
  // in slot 4); then stage 0 is complete and group 0 reads (0, 0-1)
  pp_barrier();
  pp_issue<true, true>(ld, lds + 3 * kSlotBytes, kBK, p.K, ktiles > 1);
  if (ktiles > 1)
    wait_vmcnt<kL>();
  else
    wait_vmcnt<0>();
  pp_barrier();
  v4i fa[2][C::kBI], fb[2][C::kBJ];
  if constexpr (kG == 0) {
    pp_frags<C>(lane, slot_addr(0), slot_addr(1), wrow, wcol, 0, fa, fb);
    wait_lgkm<0>();
  }
  pp_barrier();

  int sa = 0;  // slot of A_kt; B_kt is in the next one
  // kSteady: stage kt+2 exists and lies wholly below K (every load issued, none checked)
  auto iteration = [&](int kt, auto SteadyC) {
    constexpr bool kSteady = decltype(SteadyC)::value;
    const int sb = sa == kSlots - 1 ? 0 : sa + 1;
    const int na = sb == kSlots - 1 ? 0 : sb + 1;
    const int nb = na == kSlots - 1 ? 0 : na + 1;
    const int pa = sa == 0 ? kSlots - 1 : sa - 1;
    const bool more1 = kSteady || kt + 1 < ktiles, more2 = kSteady || kt + 2 < ktiles;
    const int64_t k2 = (int64_t)(kt + 2) * kBK;
    char* slot_pa = lds + pa * kSlotBytes;
    char* slot_sa = lds + sa * kSlotBytes;
    if constexpr (kG == 0) {
      pp_mma<C, 0, false>(fa, fb, acc, ld, nullptr, 0, 0, false);                       // P0
      pp_barrier();
      pp_frags<C>(lane, slot_addr(sa), slot_addr(sb), wrow, wcol, 2, fa, fb);                  // P1
      pp_issue<false, !kSteady>(ld, slot_pa, k2, p.K, more2);
      wait_lgkm<0>();
      pp_barrier();
      pp_mma<C, 0, false>(fa, fb, acc, ld, nullptr, 0, 0, false);                       // P2
    } else {
      pp_frags<C>(lane, slot_addr(sa), slot_addr(sb), wrow, wcol, 0, fa, fb);                  // P0
      pp_issue<false, !kSteady>(ld, slot_pa, k2, p.K, more2);
      wait_lgkm<0>();
      pp_barrier();
      pp_mma<C, 0, false>(fa, fb, acc, ld, nullptr, 0, 0, false);                       // P1
      pp_barrier();
      pp_frags<C>(lane, slot_addr(sa), slot_addr(sb), wrow, wcol, 2, fa, fb);                  // P2
      wait_lgkm<0>();
    }
    // stage kt+1 has landed: only A_kt+2 (when it exists) was issued after it
    if (kSteady || more2)
      wait_vmcnt<kL>();
    else
      wait_vmcnt<0>();
    pp_barrier();
    if constexpr (kG == 0) {
      // P3 (at the last stage these reads fetch slots nobody uses; they keep the code branch-free)
      pp_frags<C>(lane, slot_addr(na), slot_addr(nb), wrow, wcol, 0, fa, fb);
      pp_issue<true, !kSteady>(ld, slot_sa, k2, p.K, more2);
      wait_lgkm<0>();
    } else {
      pp_mma<C, kL, !kSteady>(fa, fb, acc, ld, slot_sa, k2, p.K, more2);                 // P3
    }
    pp_barrier();
    (void)more1;
    sa = na;
  };
  const int steady = (int)max<int64_t>(p.K / kBK - 2, 0);
  int kt = 0;
  for (; kt < steady; ++kt) iteration(kt, std::true_type{});
  before_tail();
  for (; kt < ktiles; ++kt) iteration(kt, std::false_type{});
  // Leaves with every operand load complete (the last iteration waited for all of them) and
  // every fragment read landed (each phase waits for its own), so the ring is idle; the caller
  // ends the tile with a barrier.
}

// A tile's first operand chunks: A_0, B_0 and (when K has a second stage) A_1 into slots 0-2.
template <class C>
MXQ_DEVICE void pp_first_loads(const GemmArgs& p, char* lds, const Loader<C::kLoads>& ld) {
  pp_issue<false, true>(ld, lds, 0, p.K, true);
  pp_issue<true, true>(ld, lds + C::kSlotBytes, 0, p.K, true);
  pp_issue<false, true>(ld, lds + 2 * C::kSlotBytes, kBK, p.K, p.K > kBK);
}

// One of those three chunks: A_0 (part 0), B_0 (1), A_1 (2).
template <class C>
MXQ_DEVICE void pp_first_load_part(const GemmArgs& p, char* lds, const Loader<C::kLoads>& ld, int part) {
  if (part == 0) pp_issue<false, true>(ld, lds, 0, p.K, true);
  if (part == 1) pp_issue<true, true>(ld, lds + C::kSlotBytes, 0, p.K, true);
  if (part == 2) pp_issue<false, true>(ld, lds + 2 * C::kSlotBytes, kBK, p.K, p.K > kBK);
}

// The dequant epilogues' per-tile factors, read from global memory ahead of the epilogue: the
// weight scale and the bias (raw, in the output type) of column n0 + t for thread t, and the
// per-token scales of the lane's rows. Every read is unconditional (a missing bias reads the
// first weight scale's bytes instead), so no branch waits for one.
template <int kBI, int kOut>
struct EpiFactors {
  float ws;
  typename OutT<kOut>::T bias_raw;
  float xs[kBI];
};

template <class C, int kEpi, int kOut>
MXQ_DEVICE void load_epi_factors(const GemmArgs& p, int64_t m0, int64_t n0, int wrow, EpiFactors<C::kBI, kOut>& f) {
  if constexpr (kEpi != kEpiI32) {
    typedef typename OutT<kOut>::T BT;
    const int t = tid_x(), lr = t & 31;
    const int64_t col = min(n0 + t, p.N - 1);
    f.ws = p.ws[p.ws_per_channel ? col : 0];
    f.bias_raw = *(p.bias ? reinterpret_cast<const BT*>(p.bias) + col : reinterpret_cast<const BT*>(p.ws));
#pragma unroll
    for (int i = 0; i < C::kBI; ++i) f.xs[i] = p.xs[min(m0 + wrow + i * 32 + lr, p.M - 1)];
  }
}

// The epilogue of one tile from its accumulators (lane l holds, for m-block i and n-block j, row
// wrow + i*32 + l%32 and the four column runs j*32 + q*8 + (l/32)*4 + {0..3}, q = 0..3). The LDS
// is free on entry (every wave is done with the operand ring): the per-column factors go to
// C::kEpiLds, the output staging buffers to kStageBase (table epilogues: behind the factors).
// `pre(part)`, part = 0, 1, 2 (or -1: all), issues work that must not wait for anything the epilogue does: the
// ping-pong kernel issues the next tile's first three operand chunks there, into LDS the epilogue
// does not touch (every LDS access below is inline assembly, so none of them waits for those
// loads). The parts come one before each of the first three block rows of the dequant, so that
// a wave held up issuing loads into a full memory pipeline leaves its SIMD to the other wave's
// dequant work; the gated residual epilogue, whose residual reads would wait for the loads,
// issues all three up front.
template <class C, int kEpi, int kOut, int kStageBase, int kFactorBase, class Pre>
MXQ_DEVICE void gemm_epilogue(const GemmArgs& p, char* lds, v16i (&acc)[C::kBI][C::kBJ], int64_t m0, int64_t n0,
                              int wrow, int wcol, const EpiFactors<C::kBI, kOut>& f, Pre&& pre, int pre_loads = 0) {
  constexpr int kBM = C::kBM, kBN = C::kBN, kBI = C::kBI, kBJ = C::kBJ;
  const int wave = tid_x() >> 6, lane = tid_x() & 63;
  // ---- epilogue ----
  // Lane l holds, for m-block i and n-block j, row wrow + i*32 + l%32 and the four column
  // runs j*32 + q*8 + (l/32)*4 + {0..3}, q = 0..3 (see mma_step). The main loop's last barrier
  // left the LDS free: per-column factors go to kFactorBase and, for GELU, the 128 KB
  // bf16 -> bf16 table is fetched into the ring's first slots while the dequant runs.
  constexpr int kElem = (kEpi == kEpiI32 || kOut == 0) ? 4 : 2;
  const int lr = lane & 31, lh = lane >> 5;
  const int t = tid_x();
  float* s_ws = reinterpret_cast<float*>(lds + kFactorBase);
  float* s_bias = s_ws + kBN;
  const uint16_t* s_gelu = reinterpret_cast<const uint16_t*>(lds);
  // SwiGLU: the compact SiLU table, behind the factors and the ping-pong kernel's position word
  constexpr int kSiluTabBase = kFactorBase + 2 * kBN * 4 + 2048;
  static_assert(kEpi != kEpiSwiGLU || (C::kPingPong && kSiluTabBase + 8192 <= kStageBase),
                "the SwiGLU epilogue runs in the ping-pong kernel, its table in the factors' slot");
  const bool has_b = p.bias != nullptr;
  float xsv[kBI] = {};
  if constexpr (kEpi == kEpiI32) {
  } else {
    const float bl = has_b ? OutT<kOut>::load(&f.bias_raw) : -0.0f;
    if (t < kBN) {
      lds_write_b32(lds_addr(s_ws + t), __float_as_uint(f.ws));
      lds_write_b32(lds_addr(s_bias + t), __float_as_uint(bl));
    }
    // The factors are consumed here (the row scales through an empty asm statement), before any
    // direct-to-LDS load is issued: with one of those in flight, the compiler's wait for a
    // register load is a wait for every load (vmcnt(0)). The GELU / SiLU table fetch and `pre`
    // then stay in flight through the dequant.
#pragma unroll
    for (int i = 0; i < kBI; ++i) {
      xsv[i] = f.xs[i];
      __asm__ volatile("" : "+v"(xsv[i]));
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kEpi == kEpiGelu) {
      const char* src = reinterpret_cast<const char*>(&kGeluFull) + lane * 16;
#pragma unroll 4
      for (int q = wave; q < 128; q += C::kWaves)
        __builtin_amdgcn_global_load_lds((gptr_t)(src + q * 1024), (lptr_t)(lds + q * 1024), 16, 0, 0);
    } else if constexpr (kEpi == kEpiSwiGLU) {
      // the compact SiLU table (8 KB, one kilobyte per wave) behind the factors
      static_assert(C::kWaves == 8, "one kilobyte of the compact table per wave");
      const char* src = reinterpret_cast<const char*>(&kSiluCompact) + wave * 1024 + lane * 16;
      __builtin_amdgcn_global_load_lds((gptr_t)src, (lptr_t)(lds + kSiluTabBase + wave * 1024), 16, 0, 0);
    }
    if constexpr (kEpi == kEpiGatedRes) pre(-1);  // all three parts
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt left open (max)
    barrier_no_drain();
  }
  const bool full = p.vec_store && m0 + kBM <= p.M && n0 + kBN <= p.N;
  // Interior tiles of a line-aligned output leave through LDS as whole lines (stage_store); the
  // staging buffers sit behind the per-column factors when a table fills the ring, else at 0.
  constexpr bool kTable = kEpi == kEpiGelu || kEpi == kEpiSwiGLU;
  const bool lines = full && p.line_store;
  constexpr int kSB = kEpi == kEpiGelu ? kFactorBase + 2 * kBN * 4 : kStageBase, kSE = kSB + C::kWaves * kStageBytes;
  static_assert(kSE <= C::kLds && (kSE <= kFactorBase || kSB >= kFactorBase + 2 * kBN * 4) &&
                    (kEpi != kEpiSwiGLU || kSB >= kSiluTabBase + 8192) &&
                    (kEpi != kEpiGelu || (kSB >= 128 * 1024 && kFactorBase >= 128 * 1024)),
                "staging buffers overlap the table, the factors or the end of LDS");
  char* sbuf = lds + kSB + wave * kStageBytes;
  const int64_t pitch = p.ldd * kElem;
  int64_t grow[kBI] = {};     // kEpiGatedRes: the gate row of each of this lane's rows
  int64_t grow_rm[kBI][4] = {};  // ... and of the rows it updates in the whole-line form
  if constexpr (kEpi == kEpiGatedRes) {
    auto gate_row = [&](int64_t m) {  // clamped into the gate so a bad row index cannot fault
      const int64_t gr = p.gate_rows[min(m, p.M - 1)];
      return gr < 0 ? (int64_t)0 : (gr >= p.gate_count ? p.gate_count - 1 : gr);
    };
#pragma unroll
    for (int i = 0; i < kBI; ++i) {
      grow[i] = gate_row(m0 + wrow + i * 32 + lr);
      if (lines)
#pragma unroll
        for (int t = 0; t < 4; ++t) grow_rm[i][t] = gate_row(m0 + wrow + i * 32 + t * 8 + (lane >> 3));
    }
  }

  // The blocks go by pairs of 32-column blocks (jp), the factors of a pair held in registers; an
  // odd last block (128 x 96 tiles: three blocks per wave) goes alone, with run stores.
  // GELU / SwiGLU: pre-activation bf16 pairs, kept until the table has landed.
  static_assert(!kTable || kBJ % 2 == 0, "the table epilogues take pairs of blocks");
  uint32_t yp[kTable ? kBI : 1][kTable ? kBJ : 1][8];
  static_for<(kBJ + 1) / 2>([&](auto JP) {
    constexpr int jp = decltype(JP)::value;
    constexpr int kJJ = 2 * jp + 2 <= kBJ ? 2 : 1;  // blocks in this group
    float wsv[2][16], bsv[2][16];
    if constexpr (kEpi != kEpiI32) {
      // columns wcol + (2 jp + jj) * 32 + lh * 4 + q * 8 + {0..3}
      const uint32_t a_ws = lds_addr(s_ws + wcol + 2 * jp * 32 + lh * 4), a_b = a_ws + kBN * 4;
      v4i w4[2][4], b4[2][4];
      static_for<kJJ>([&](auto JJ) {
        static_for<4>([&](auto Q) {
          constexpr int kOff = decltype(JJ)::value * 128 + decltype(Q)::value * 32;
          w4[decltype(JJ)::value][decltype(Q)::value] = lds_read_b128<kOff>(a_ws);
          b4[decltype(JJ)::value][decltype(Q)::value] = lds_read_b128<kOff>(a_b);
        });
      });
      wait_lgkm<0>();
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int jj = 0; jj < kJJ; ++jj)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            wsv[jj][q * 4 + e] = __int_as_float(w4[jj][q][e]);
            bsv[jj][q * 4 + e] = __int_as_float(b4[jj][q][e]);
          }
    }
    static_for<kBI>([&](auto I) {
      constexpr int i = decltype(I)::value;
      if constexpr (kEpi != kEpiGatedRes && jp == 0 && i < 3) {
        __builtin_amdgcn_sched_barrier(0);
        pre(i);
        __builtin_amdgcn_sched_barrier(0);
      }
      constexpr int kWords = kElem == 4 ? 4 : 2;
      const int64_t row0 = m0 + wrow + i * 32;  // the block row's first row
      const int64_t col0 = n0 + wcol + jp * 64;  // the pair's first column
      uint32_t w[2][8];
      uint32_t w32[2][16];
#pragma unroll
      for (int jj = 0; jj < kJJ; ++jj)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if constexpr (kElem == 4)
            epi_run<kEpi, kOut>(acc[i][2 * jp + jj], q, xsv[i], wsv[jj] + q * 4, bsv[jj] + q * 4, w32[jj] + q * kWords);
          else
            epi_run<kEpi, kOut>(acc[i][2 * jp + jj], q, xsv[i], wsv[jj] + q * 4, bsv[jj] + q * 4, w[jj] + q * kWords);
        }
      if constexpr (kTable) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
#pragma unroll
          for (int r = 0; r < 8; ++r) yp[i][2 * jp + jj][r] = w[jj][r];
      } else if constexpr (kEpi == kEpiGatedRes) {
        if (lines && kJJ == 2) {
          gated_lines(p, sbuf, row0, col0, grow_rm[i], w);
        } else {
#pragma unroll
          for (int jj = 0; jj < kJJ; ++jj) gated_block_row(p, full, row0 + lr, grow[i], col0 + jj * 32 + lh * 4, w[jj]);
        }
      } else if constexpr (kElem == 4) {
        if (lines) {
#pragma unroll
          for (int jj = 0; jj < kJJ; ++jj) {
            stage_block32(sbuf, w32[jj]);
            stage_store(p, sbuf, row0, (col0 + jj * 32) * 4, pitch);
          }
        } else {
#pragma unroll
          for (int jj = 0; jj < kJJ; ++jj) store_block_row<4>(p, full, row0 + lr, col0 + jj * 32 + lh * 4, w32[jj]);
        }
      } else {
        if (lines && kJJ == 2) {
          stage_blocks16(sbuf, w);
          stage_store(p, sbuf, row0, col0 * 2, pitch);
        } else {
#pragma unroll
          for (int jj = 0; jj < kJJ; ++jj) store_block_row<2>(p, full, row0 + lr, col0 + jj * 32 + lh * 4, w[jj]);
        }
      }
    });
  });
  if constexpr (kEpi == kEpiGelu) {
    typedef unsigned short us2 __attribute__((ext_vector_type(2)));
    wait_vmcnt<0>();
    barrier_no_drain();  // every wave's part of the table has landed
    // |h| as bf16 bits: non-negative values order like their bit patterns (NaN above +inf), so
    // the row maximum is an integer maximum, kept for both halves of a word at once.
    us2 rmax[kBI] = {};
    // kMode 2: interior tile, whole-line stores; 1: interior tile, run stores; 0: edge tile,
    // column masks and store guards.
    auto gelu_pass = [&](auto ModeC) {
      constexpr int kMode = decltype(ModeC)::value;
      static_for<kBI>([&](auto I) {
        constexpr int i = decltype(I)::value;
        const int64_t row0 = m0 + wrow + i * 32;
        static_for<kBJ / 2>([&](auto JP) {
          constexpr int jp = decltype(JP)::value;
          const int64_t col0 = n0 + wcol + jp * 64;
          uint32_t g[2][8];
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) {
#pragma unroll
            for (int r = 0; r < 8; ++r) {
              const uint32_t h = yp[i][2 * jp + jj][r];
              g[jj][r] = (uint32_t)s_gelu[h & 0xFFFFu] | ((uint32_t)s_gelu[h >> 16] << 16);
            }
#pragma unroll
            for (int r = 0; r < 8; ++r) {
              uint32_t m = g[jj][r] & 0x7FFF7FFFu;
              if constexpr (kMode == 0) {
                const int64_t col = col0 + jj * 32 + lh * 4 + (r >> 1) * 8 + (r & 1) * 2;
                m &= (col < p.N ? 0xFFFFu : 0u) | (col + 1 < p.N ? 0xFFFF0000u : 0u);
              }
              rmax[i] = __builtin_elementwise_max(rmax[i], __builtin_bit_cast(us2, m));
            }
          }
          if constexpr (kMode == 2) {
            stage_blocks16(sbuf, g);
            stage_store(p, sbuf, row0, col0 * 2, pitch);
          } else {
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) store_block_row<2>(p, kMode == 1, row0 + lr, col0 + jj * 32 + lh * 4, g[jj]);
          }
        });
      });
    };
    if (lines)
      gelu_pass(std::integral_constant<int, 2>{});
    else if (full)
      gelu_pass(std::integral_constant<int, 1>{});
    else
      gelu_pass(std::integral_constant<int, 0>{});
    // Lanes l and l + 32 hold the two halves of each row's columns of this wave.
#pragma unroll
    for (int i = 0; i < kBI; ++i) {
      uint32_t m = max((uint32_t)rmax[i][0], (uint32_t)rmax[i][1]);
      m = max(m, (uint32_t)__shfl_xor((int)m, 32, kWave));
      const int64_t row = m0 + wrow + i * 32 + lr;
      if (lh == 0 && row < p.M) atomicMax(reinterpret_cast<unsigned int*>(p.row_absmax + row), m << 16);
    }
  }
  if constexpr (kEpi == kEpiSwiGLU) {
    // Every wave's kilobyte of the SiLU table has landed: only the `pre_loads` loads of the next
    // tile, issued after it, may stay in flight (a wait for more than those is still correct).
    if (pre_loads >= 3 * C::kLoads)
      wait_vmcnt<3 * C::kLoads>();
    else if (pre_loads >= 2 * C::kLoads)
      wait_vmcnt<2 * C::kLoads>();
    else if (pre_loads >= C::kLoads)
      wait_vmcnt<C::kLoads>();
    else
      wait_vmcnt<0>();
    barrier_no_drain();
    // Runs 0, 1 of a 32 x 32 block are gate columns, runs 2, 3 the matching up columns; output
    // channel c of block b (tile column t0 = b * 32) is h column t0 / 2 + c. A wave's blocks of a
    // block row give 16 h columns each: a 64-byte piece per row (two blocks) for the whole-line
    // form, or a 128-byte one (four).
    const uint32_t tab = lds_addr(lds + kSiluTabBase);
    const int64_t nh = p.N / 2;
    const bool hfull = p.vec_store && m0 + kBM <= p.M && (n0 + kBN) / 2 <= nh;
    const bool hlines = hfull && p.line_store;
    static_for<kBI>([&](auto I) {
      constexpr int i = decltype(I)::value;
      const int64_t row = m0 + wrow + i * 32 + lr;
      uint32_t hw[kBJ][4];
      // silu of the row's gate values from the compact table (LDS reads as inline assembly: the
      // next tile's operand loads stay in flight), then the rules for values outside its range
      uint32_t sg[kBJ][4][2];
#pragma unroll
      for (int j = 0; j < kBJ; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t g = yp[i][j][r];
          sg[j][r][0] = lds_read_u16_at(tab + silu_compact_offset(g & 0xFFFFu));
          sg[j][r][1] = lds_read_u16_at(tab + silu_compact_offset(g >> 16));
        }
      wait_lgkm<0>();
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < kBJ; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t g = yp[i][j][r], u = yp[i][j][r + 4];
          const uint32_t glo = g & 0xFFFFu, ghi = g >> 16;
          const uint32_t slo = silu_compact_in(glo) ? sg[j][r][0] : silu_rule_out(glo);
          const uint32_t shi = silu_compact_in(ghi) ? sg[j][r][1] : silu_rule_out(ghi);
          const float plo = bf16_to_f32(slo) * bf16_to_f32(u & 0xFFFFu);
          const float phi = bf16_to_f32(shi) * bf16_to_f32(u >> 16);
          hw[j][r] = (plo != plo ? 0x7FC0u : f32_to_bf16_bits(plo)) | ((phi != phi ? 0x7FC0u : f32_to_bf16_bits(phi)) << 16);
        }
      if (hlines) {
        wave_lds_sync();
#pragma unroll
        for (int j = 0; j < kBJ; ++j) {
          stage_put8(sbuf, lr, j * 2, lh, hw[j][0], hw[j][1]);
          stage_put8(sbuf, lr, j * 2 + 1, lh, hw[j][2], hw[j][3]);
        }
        if constexpr (kBJ == 4)
          stage_store(p, sbuf, m0 + wrow + i * 32, (n0 + wcol) / 2 * 2, pitch);
        else
          stage_store64(p, sbuf, m0 + wrow + i * 32, (n0 + wcol) / 2 * 2, pitch);
      } else {
#pragma unroll
        for (int j = 0; j < kBJ; ++j) {
          const int64_t hc0 = (n0 + wcol + j * 32) / 2 + lh * 4;
          if (hfull || row < p.M) {
            store_run<2>(p.d, p.ldd, row, hc0, nh, hfull || (p.vec_store && hc0 + 4 <= nh), hw[j]);
            store_run<2>(p.d, p.ldd, row, hc0 + 8, nh, hfull || (p.vec_store && hc0 + 12 <= nh), hw[j] + 2);
          }
        }
      }
    });
  }
}

// ---- persistent ping-pong workgroups ----
// With the tile queue, the ping-pong kernel runs W = wg_per_xcd workgroups per XCD (one per CU)
// that loop over tiles. XCD x's range splits as in pick_tile: its first count_x - pool positions
// are static, its last `pool` are claimed at run time. Workgroup (x = bid % 8, k = bid / 8) takes
// the static positions start_x + k, start_x + k + W, ... and then claims pool positions, from its
// own XCD's counter first and then from the others in turn; a counter found drained is not asked
// again (nothing refills it during a launch). Only the last eighth of the tiles thus waits for a
// claim, and no claim is in flight across a main loop (the vmcnt waits there count operand loads
// only). Wave 0 decides the next position (lane 0 claims, the wave reads the result as a scalar,
// so the claim state costs no vector registers) and passes it to the workgroup through LDS. A
// workgroup that finds every counter drained counts itself out (acquire-release); the last one
// of the launch resets the counters for the next.
MXQ_DEVICE int pp_claim(const GemmArgs& p, int num, int& j) {
  const int x = blockIdx.x & 7;
  const bool lane0 = (tid_x() & 63) == 0;
  for (; j < 8; ++j) {
    const int y = (x + j) & 7;
    unsigned i = 0;
    if (lane0) i = __hip_atomic_fetch_add(p.counters + y * 32, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    i = (unsigned)__builtin_amdgcn_readfirstlane((int)i);
    if (i < (unsigned)p.pool) {
      int ys, yc;
      xcd_range(y, num, ys, yc);
      return ys + yc - p.pool + (int)i;
    }
  }
  // Release: this workgroup's claims are ordered before its count; acquire: the last one sees
  // every claim of the launch (the counts form one release sequence) before it resets.
  if (lane0) {
    const unsigned done = __hip_atomic_fetch_add(p.counters + 8 * 32, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (done == (unsigned)p.n_claim - 1) {
      for (int y = 0; y < 8; ++y) __hip_atomic_exchange(p.counters + y * 32, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_exchange(p.counters + 8 * 32, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  return -1;
}

// The ping-pong kernel: its tiles (one, or a sequence when p.persistent), each through the main
// loop and the epilogue. LDS at tile boundaries: slots 0-2 take the next tile's first chunks while
// the epilogue keeps its per-column factors in slot 3 and its output staging in slot 4; the next
// position passes from wave 0 to the workgroup through a word of slot 3.
template <class C, int kEpi, int kOut>
MXQ_DEVICE void pp_tiles(const GemmArgs& p, char* lds) {
  static_assert(C::kWaves == 8 && C::kSlots == 5 && C::kLoads == 4, "the ping-pong ring");
  constexpr int kSlotBytes = C::kSlotBytes, kFactorBase = 3 * kSlotBytes, kStageBase = 4 * kSlotBytes;
  static_assert(kFactorBase + 2 * C::kBN * 4 + 4 <= kStageBase, "slot 3 holds the factors and the next position");
  const uint32_t next_word = lds_addr(lds + kFactorBase + 2 * C::kBN * 4);
  const int num = p.tiles_m * p.tiles_n;
  const bool wave0 = __builtin_amdgcn_readfirstlane(tid_x() >> 6) == 0;
  // Wave 0's next position: the next static one while there is one, then claims; -1 at the end.
  int static_next = -1, static_end = 0, claim_j = 0;
  auto next_position = [&]() -> int {
    if (!p.persistent) return -1;
    if (static_next >= 0 && static_next < static_end) {
      const int pos = static_next;
      static_next += p.wg_per_xcd;
      return pos;
    }
    static_next = -1;
    return pp_claim(p, num, claim_j);
  };
  int pos;
  if (p.persistent) {
    int s, c;
    xcd_range(blockIdx.x & 7, num, s, c);
    static_next = s + (int)(blockIdx.x >> 3);
    static_end = s + c - p.pool;
    if (static_next < static_end) {
      pos = static_next;
      static_next += p.wg_per_xcd;
    } else {  // more workgroups than static positions: the first tile is claimed too
      if (wave0) {
        const int got = next_position();
        if ((tid_x() & 63) == 0) lds_write_b32(next_word, (uint32_t)got);
      }
      wait_all();
      pp_barrier();
      const uint32_t r = lds_read_b32(next_word);
      wait_lgkm<0>();
      __builtin_amdgcn_sched_barrier(0);
      pos = __builtin_amdgcn_readfirstlane((int)r);
      pp_barrier();  // read before the first loads land in slot 3's neighbourhood
      if (pos < 0) return;
    }
  } else {
    pos = pick_tile(p, num, lds);
    if (pos < 0) return;
  }
  const int wave = __builtin_amdgcn_readfirstlane(tid_x() >> 6);  // scalar: so are wrow and wcol
  // The wave's first output row and column in the tile: the two waves of a SIMD (w and w + 4)
  // take the two 64-column halves of 128 x 128 quadrant w of the 2 x 2 grid.
  const int wrow = ((wave & 3) >> 1) * C::kWaveM;
  const int wcol = (wave & 1) * 128 + (wave >> 2) * 64;
  const bool group0 = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 8)) == 0;
  int tm, tn;
  tile_walk(pos, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
  int64_t m0 = (int64_t)tm * C::kBM, n0 = (int64_t)tn * C::kBN;
  {
    Loader<C::kLoads> first;
    make_loader(first, p, m0, n0);
    pp_first_loads<C>(p, lds, first);
  }
  for (;;) {
    // (formed again per tile: the next tile's first loads use a copy of their own, so no loader
    // stays live through the epilogue)
    Loader<C::kLoads> ld;
    make_loader(ld, p, m0, n0);
    v16i acc[C::kBI][C::kBJ];
#pragma unroll
    for (int i = 0; i < C::kBI; ++i)
#pragma unroll
      for (int j = 0; j < C::kBJ; ++j) acc[i][j] = v16i{};
    EpiFactors<C::kBI, kOut> f;
    auto factors = [&] { load_epi_factors<C, kEpi, kOut>(p, m0, n0, wrow, f); };
    if (group0)
      pp_loop<C, 0>(p, lds, acc, wrow, wcol, ld, factors);
    else
      pp_loop<C, 1>(p, lds, acc, wrow, wcol, ld, factors);
    // The ring is idle (pp_loop): slot 3 takes the next position before the barrier that ends
    // the tile publishes it.
    if (wave0) {
      const int got = next_position();
      if ((tid_x() & 63) == 0) lds_write_b32(next_word, (uint32_t)got);
    }
    wait_all();
    pp_barrier();
    const uint32_t next_read = lds_read_b32(next_word);
    wait_lgkm<0>();
    __builtin_amdgcn_sched_barrier(0);
    const int next = __builtin_amdgcn_readfirstlane((int)next_read);
    int64_t nm0 = 0, nn0 = 0;
    gemm_epilogue<C, kEpi, kOut, kStageBase, kFactorBase>(p, lds, acc, m0, n0, wrow, wcol, f, [&](int part) {
      if (next >= 0) {
        if (part <= 0) {  // the first call
          int ntm, ntn;
          tile_walk(next, p.tiles_m, p.tiles_n, p.group_m, ntm, ntn);
          nm0 = (int64_t)ntm * C::kBM;
          nn0 = (int64_t)ntn * C::kBN;
        }
        // (a loader formed per part: one kept live through the epilogue would take registers)
        Loader<C::kLoads> next_ld;
        make_loader(next_ld, p, nm0, nn0);
        if (part < 0)
          pp_first_loads<C>(p, lds, next_ld);
        else
          pp_first_load_part<C>(p, lds, next_ld, part);
      }
    }, next >= 0 ? (p.K > kBK ? 3 : 2) * C::kLoads : 0);
    if (next < 0) break;
    m0 = nm0;
    n0 = nn0;
  }
}

// The four-wave kernels: one tile per workgroup.
template <class C, int kEpi, int kOut>
MXQ_DEVICE void four_wave_tile(const GemmArgs& p, char* lds) {
  constexpr int kBM = C::kBM, kBN = C::kBN, kWaveM = C::kWaveM, kWaveN = C::kWaveN;
  constexpr int kBI = C::kBI, kBJ = C::kBJ, kSlotBytes = C::kSlotBytes, kLoads = C::kLoads;
  constexpr int kSlots = C::kSlots, kAhead = C::kAhead;
  constexpr int kStageLoads = C::kLoads + C::kLoadsB;  // loads per wave per stage (A and B chunks)
  const int pos = pick_tile(p, p.tiles_m * p.tiles_n, lds);
  if (pos < 0) return;
  int tm, tn;
  tile_walk(pos, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
  const int64_t m0 = (int64_t)tm * kBM, n0 = (int64_t)tn * kBN;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // The wave's first output row and column in the tile: a 2 x 2 grid of quadrants (128 x 96
  // tiles: four 32-row strips).
  const int wrow = (wave / C::kWavesN) * kWaveM;
  const int wcol = (wave % C::kWavesN) * kWaveN;

  v16i acc[kBI][kBJ];
#pragma unroll
  for (int i = 0; i < kBI; ++i)
#pragma unroll
    for (int j = 0; j < kBJ; ++j) acc[i][j] = v16i{};

  {
    // Pipeline (D = kAhead stages ahead, a ring of S = 2D + 1 slots of one operand chunk each):
    // the operand chunks arrive in the order A0 B0 A1 B1 A2 ..., chunk i (A_j = 2j, B_j = 2j + 1)
    // into slot i % S; stage j (128 K-bytes) reads A_j and B_j. Entering iteration kt, A_kt and
    // B_kt are complete and visible, stages kt+1 .. kt+D-1 are in flight and F0 holds the
    // fragments of (stage kt, K-step 0). The iteration runs K-steps 0..3, each step's fragments
    // read behind the previous step's MFMAs. A_kt+D goes into the slot of B_kt-1 (free since the
    // previous barrier) with its loads spread over the MFMAs of K-steps 0 and 1; before the MFMAs
    // of K-step 3 the wave waits for stage kt+1, passes the barrier that frees the slots of A_kt
    // and B_kt, reads (kt+1, 0), and spreads the loads of B_kt+D over those MFMAs (into A_kt's
    // slot). A chunk is thus requested D-1 to D stages before it is used, and no wave issues a
    // burst of loads while its matrix pipe sits idle.
    const int ktiles = (int)((p.K + kBK - 1) / kBK);
    Loader<kLoads, C::kLoadsB> ld;
    make_loader(ld, p, m0, n0);
    const int pre = min(ktiles, kAhead);  // stages requested before the loop
    for (int s = 0; s < pre; ++s) {
      issue_slot<false>(ld, lds + 2 * s * kSlotBytes, (int64_t)s * kBK, p.K);
      issue_slot<true>(ld, lds + (2 * s + 1) * kSlotBytes, (int64_t)s * kBK, p.K);
    }
    // wait for stage 0: every load but those of stages 1 .. pre-1 has completed
    static_for<kAhead>([&](auto P) {
      constexpr int np = decltype(P)::value + 1;
      if (pre == np) wait_vmcnt<(np - 1) * kStageLoads>();
    });
    barrier_no_drain();

    const uint32_t lds_addr = (uint32_t)(uintptr_t)(lptr_t)lds;
    v4i f0a[kBI], f0b[kBJ], f1a[kBI], f1b[kBJ];
    load_frags<C>(lane, lds_addr, lds_addr + kSlotBytes, wrow, wcol, 0, f0a, f0b);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_sched_barrier(0);
    int sa = 0;  // slot of A_kt; B_kt is in (sa + 1) % 5
    // One iteration. kSteady: stage kt+2 exists and lies wholly below K, so every load of the
    // iteration is issued and none needs the K-tail check (no per-load compare, select or branch);
    // the last two or three iterations take the general form.
    auto iteration = [&](int kt, auto steady) {
      constexpr bool kSteady = decltype(steady)::value;
      const int sb = sa == kSlots - 1 ? 0 : sa + 1;
      const int na = sb == kSlots - 1 ? 0 : sb + 1;  // A_kt+1
      const int nb = na == kSlots - 1 ? 0 : na + 1;  // B_kt+1
      const int pa = sa == 0 ? kSlots - 1 : sa - 1;  // A_kt+D (slot of B_kt-1)
      const uint32_t cur_a = lds_addr + (uint32_t)(sa * kSlotBytes), cur_b = lds_addr + (uint32_t)(sb * kSlotBytes);
      const bool more2 = kSteady || kt + kAhead < ktiles;  // stage kt+D exists
      const bool more1 = kSteady || kt + 1 < ktiles;
      const int64_t k2 = (int64_t)(kt + kAhead) * kBK;
      load_frags<C>(lane, cur_a, cur_b, wrow, wcol, 1, f1a, f1b);
      wait_lgkm<kBI + kBJ>();
      __builtin_amdgcn_sched_barrier(0);
      mma_step_dma<C, false, 0, kLoads / 2, !kSteady>(f0a, f0b, acc, ld, lds + pa * kSlotBytes, k2, p.K, more2);
      __builtin_amdgcn_sched_barrier(0);
      load_frags<C>(lane, cur_a, cur_b, wrow, wcol, 2, f0a, f0b);
      wait_lgkm<kBI + kBJ>();
      __builtin_amdgcn_sched_barrier(0);
      mma_step_dma<C, false, kLoads / 2, kLoads / 2, !kSteady>(f1a, f1b, acc, ld, lds + pa * kSlotBytes, k2, p.K, more2);
      __builtin_amdgcn_sched_barrier(0);
      load_frags<C>(lane, cur_a, cur_b, wrow, wcol, 3, f1a, f1b);
      wait_lgkm<kBI + kBJ>();
      __builtin_amdgcn_sched_barrier(0);
      mma_step<C>(f0a, f0b, acc);
      __builtin_amdgcn_sched_barrier(0);
      // Stage kt+1 has landed when only the loads issued after B_kt+1 are outstanding: stages
      // kt+2 .. kt+D-1 and A_kt+D where they exist (2 (r - 1) chunks when only r < D stages remain).
      if (more2) {
        wait_vm_lgkm0<(kAhead - 2) * kStageLoads + kLoads>();
      } else if constexpr (kAhead > 2) {
        const int r = ktiles - 1 - kt;
        if (r == 3) {
          wait_vm_lgkm0<2 * kStageLoads>();
        } else if (r == 2) {
          wait_vm_lgkm0<kStageLoads>();
        } else {
          wait_all();
        }
      } else {
        wait_all();
      }
      __builtin_amdgcn_sched_barrier(0);
      if (more1) {
        barrier_no_drain();
        load_frags<C>(lane, lds_addr + (uint32_t)(na * kSlotBytes), lds_addr + (uint32_t)(nb * kSlotBytes), wrow, wcol, 0, f0a, f0b);
      }
      __builtin_amdgcn_sched_barrier(0);
      mma_step_dma<C, true, 0, C::kLoadsB, !kSteady>(f1a, f1b, acc, ld, lds + sa * kSlotBytes, k2, p.K, more2 && more1);
      __builtin_amdgcn_sched_barrier(0);
      sa = na;
    };
    // steady < ktiles always (ktiles >= 1): written as do-while, the tail is seen to run at least
    // once, so no path leaves the steady loop with fragment reads in flight straight into the
    // epilogue (whose register copies would otherwise race those reads).
    const int steady = (int)max<int64_t>(p.K / kBK - kAhead, 0);  // iterations whose stage kt+D is full
    int kt = 0;
    for (; kt < steady; ++kt) iteration(kt, std::true_type{});
    do {
      iteration(kt, std::false_type{});
    } while (++kt < ktiles);
    // Every wave is done reading the ring before the epilogue reuses it, and the last (unused)
    // fragment reads have landed before their registers are reused.
    wait_all();
    __builtin_amdgcn_sched_barrier(0);
    barrier_no_drain();
  }

  EpiFactors<kBI, kOut> f;
  load_epi_factors<C, kEpi, kOut>(p, m0, n0, wrow, f);
  gemm_epilogue<C, kEpi, kOut, 0, C::kEpiLds>(p, lds, acc, m0, n0, wrow, wcol, f, [](int) {});
}

template <int kEpi, int kOut, int kT, bool kDeep, bool kPP, int kTN = kT>
__global__ __launch_bounds__((TileCfg<kT, kDeep, kPP, kTN>::kThreads), (TileCfg<kT, kDeep, kPP, kTN>::kPerCu)) void gemm_i8_kernel(GemmArgs p) {
  typedef TileCfg<kT, kDeep, kPP, kTN> C;
  static_assert(kT == 256 || (kEpi != kEpiGelu && kEpi != kEpiSwiGLU), "table epilogues need the 160 KB ring");
  __shared__ __attribute__((aligned(16))) char lds[C::kLds];
  if constexpr (kPP)
    pp_tiles<C, kEpi, kOut>(p, lds);
  else
    four_wave_tile<C, kEpi, kOut>(p, lds);
}

// Balanced tile queue (pick_tile): each XCD's pool is 1/kPoolDiv of its range and each XCD
// gets as many extra workgroups as its pool holds tiles; problems of fewer than two rounds of
// tiles keep the static order.
constexpr int kPoolDiv = 8;
constexpr int kTileQueueBytes = 9 * 128;  // 8 pool counters and the claim count, a line each
static_assert(MXQ_GEMM_WORKSPACE_BYTES >= kTileQueueBytes, "workspace holds the tile queue counters");

// Launch plan of one GEMM: tile size, tile queue and grid.
struct GemmPlan {
  int tile;  // 256 or 128 (rows of a tile)
  int tile_n;  // columns of a tile: the tile size, or 96 (128 x 96 deep-ring tiles)
  bool deep;  // 128-tiles with the deep ring: every tile on its own CU at once
  int tiles_m, tiles_n;
  int pool, wg_per_xcd, n_claim;
  int group_m;
  int64_t grid;
  bool persistent;  // ping-pong workgroups that loop over their XCD's tiles (pp_tiles)
};

// Problems with fewer 256-tiles than CUs run 128-tiles (four times as many workgroups). Larger ones
// run 128-tiles too when their rounds finish first: 256 CUs hold 256 workgroups of 256-tiles or 512
// of 128-tiles, and a round of 128-tiles takes about 0.55 of a round of 256-tiles (measured at
// K = 4096-8192), so a last round of 256-tiles that is mostly empty is cheaper as 128-tiles
// (4096 x 5120: 1.25 rounds, 0.147 -> 0.117 ms) and a full one is not. The table epilogues (GELU,
// SwiGLU) need the 256-tile ring. With a workspace, problems of two rounds or more balance their
// tiles over the XCDs at run time (pick_tile).
static GemmPlan plan_gemm(int64_t M, int64_t N, int table, int64_t workspace_bytes) {
  GemmPlan g{};
  const int64_t big_tiles = ((M + 255) / 256) * ((N + 255) / 256);
  const int64_t tiles128 = ((M + 127) / 128) * ((N + 127) / 128);
  const bool prefer128 = big_tiles < 256 || ((tiles128 + 511) / 512) * 11 < ((big_tiles + 255) / 256) * 20;
  g.tile = !table && prefer128 ? 128 : 256;
  g.deep = g.tile == 128 && tiles128 <= 256;
  // Deep-ring problems whose 128 x 96 tiles still fit on the CUs at once take those: more CUs,
  // each with three quarters of the work (1024 x 3072: 256 tiles instead of 192).
  const int64_t tiles96 = ((M + 127) / 128) * ((N + 95) / 96);
  g.tile_n = g.deep && tiles96 > tiles128 && tiles96 <= std::min(mxq_cu_count(), 256) ? 96 : g.tile;
  g.tiles_m = (int)std::min<int64_t>((M + g.tile - 1) / g.tile, INT32_MAX);
  g.tiles_n = (int)std::min<int64_t>((N + g.tile_n - 1) / g.tile_n, INT32_MAX);
  const int64_t tiles = (int64_t)g.tiles_m * g.tiles_n;
  g.grid = tiles;
  // Deep-ring problems run every tile at once, one per CU: each XCD fetches the A and B panels
  // of its range once, so the range is made as square as the groups allow (1024 x 3072, 24
  // tiles per XCD: 4 x 6 tiles read 10 panels where 2 x 12 read 14; 17.8 against 18.5 us per
  // launch with operands from HBM). Two workgroups per CU measured no better this way.
  g.group_m = g.tile == 256 && table != kTableGelu ? kGroupMPingPong : kGroupM;
  const int64_t slots = g.tile == 256 ? 256 : 512;
  if (g.deep) {
    const int64_t per = (tiles + 7) / 8;
    int64_t best = INT64_MAX;
    for (int64_t gm = 1; gm <= std::min<int64_t>(g.tiles_m, per); ++gm) {
      const int64_t panels = gm + (per + gm - 1) / gm;
      if (panels < best) {
        best = panels;
        g.group_m = (int)gm;
      }
    }
  }
  if (workspace_bytes >= kTileQueueBytes && tiles >= 2 * slots && tiles <= INT32_MAX / 2) {
    const int64_t per = tiles / 8, rem = tiles % 8;
    g.pool = (int)((per + kPoolDiv - 1) / kPoolDiv);
    if (g.tile == 256 && table != kTableGelu) {
      // Ping-pong tiles: one workgroup per CU, each looping over its XCD's static positions and
      // then over claimed ones, so that a tile's epilogue overlaps the next tile's first loads.
      g.persistent = true;
      g.wg_per_xcd = std::max(1, mxq_cu_count() / 8);
      g.grid = 8 * (int64_t)g.wg_per_xcd;
      g.n_claim = (int)g.grid;
    } else {
      g.wg_per_xcd = (int)(per + (rem ? 1 : 0) + g.pool);
      g.grid = 8 * (int64_t)g.wg_per_xcd;
      g.n_claim = (int)(g.grid - tiles + 8 * (int64_t)g.pool);
    }
  }
  return g;
}

template <int kEpi, int kOut>
static int launch_gemm(const GemmArgs& args0, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  GemmArgs args = args0;
  const GemmPlan g = plan_gemm(args.M, args.N, kEpi == kEpiGelu ? kTableGelu : kEpi == kEpiSwiGLU ? kTableSwiGLU : 0,
                               workspace ? workspace_bytes : 0);
  if ((int64_t)g.tiles_m * g.tiles_n > INT32_MAX / 2) return mxq_set_error(MXQ_ERR_UNSUPPORTED, "too many tiles");
  args.tiles_m = g.tiles_m;
  args.tiles_n = g.tiles_n;
  args.pool = g.pool;
  args.wg_per_xcd = g.wg_per_xcd;
  args.n_claim = g.n_claim;
  args.counters = g.pool ? reinterpret_cast<unsigned*>(workspace) : nullptr;
  args.group_m = g.group_m;
  args.persistent = g.persistent;
  const int elem = (kOut == 0 || kEpi == kEpiI32) ? 4 : 2;
  args.vec_store = ((uintptr_t)args.d % (4 * elem) == 0) && (args.ldd % 4 == 0);
  args.line_store = ((uintptr_t)args.d % 16 == 0) && ((args.ldd * elem) % 16 == 0);
  if (kEpi == kEpiGatedRes) {
    args.vec_store = args.vec_store && ((uintptr_t)args.gate % 8 == 0) && (args.ldg % 4 == 0);
    args.line_store = args.line_store && ((uintptr_t)args.gate % 16 == 0) && (args.ldg % 8 == 0);
  }
  const unsigned grid = (unsigned)g.grid;
  if constexpr (kEpi == kEpiSwiGLU) {
    // 256-tiles on the ping-pong schedule, the compact SiLU table in the epilogue
    gemm_i8_kernel<kEpi, kOut, 256, false, true><<<grid, TileCfg<256, false, true>::kThreads, 0, stream>>>(args);
  } else if constexpr (kEpi != kEpiGelu) {
    if (g.tile == 128) {
      if (g.deep && g.tile_n == 96)
        gemm_i8_kernel<kEpi, kOut, 128, true, false, 96><<<grid, kGemmThreads, 0, stream>>>(args);
      else if (g.deep)
        gemm_i8_kernel<kEpi, kOut, 128, true, false><<<grid, kGemmThreads, 0, stream>>>(args);
      else
        gemm_i8_kernel<kEpi, kOut, 128, false, false><<<grid, kGemmThreads, 0, stream>>>(args);
      return mxq_check_launch("gemm_i8_kernel");
    }
    // 256-tiles without a table epilogue: the ping-pong schedule (eight waves)
    gemm_i8_kernel<kEpi, kOut, 256, false, true><<<grid, TileCfg<256, false, true>::kThreads, 0, stream>>>(args);
  } else {
    gemm_i8_kernel<kEpi, kOut, 256, false, false><<<grid, kGemmThreads, 0, stream>>>(args);
  }
  return mxq_check_launch("gemm_i8_kernel");
}

// The tile-queue workspace: NULL (static order) or 256-byte aligned.
static int check_workspace(const void* workspace, int64_t workspace_bytes) {
  if (!workspace) return MXQ_OK;
  if (workspace_bytes < 0) return mxq_set_error(MXQ_ERR_INVALID, "negative workspace size");
  if ((uintptr_t)workspace % 256) return mxq_set_error(MXQ_ERR_INVALID, "GEMM workspace must be 256-byte aligned");
  return MXQ_OK;
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

extern "C" int mxq_int8_gemm_plan(int64_t M, int64_t N, int64_t K, int table_epilogue,
                                  int64_t workspace_bytes, int64_t* plan) {
  if (M <= 0 || N <= 0 || K <= 0 || !plan) return mxq_set_error(MXQ_ERR_INVALID, "GEMM plan needs a positive shape and an output");
  if (table_epilogue < 0 || table_epilogue > kTableSwiGLU) return mxq_set_error(MXQ_ERR_INVALID, "table_epilogue must be 0, 1 or 2");
  const GemmPlan g = plan_gemm(M, N, table_epilogue, workspace_bytes);
  plan[0] = g.tile;
  plan[1] = g.grid;
  plan[2] = (int64_t)g.tiles_m * g.tiles_n;
  plan[3] = g.pool;
  plan[4] = g.wg_per_xcd;
  plan[5] = g.tile == 256 ? TileCfg<256>::kAhead : g.deep ? TileCfg<128, true>::kAhead : TileCfg<128>::kAhead;
  plan[6] = g.group_m;
  plan[7] = g.persistent;
  plan[8] = g.tile_n;
  return MXQ_OK;
}

extern "C" int mxq_int8_gemm_i32(const int8_t* a, const int8_t* b, int32_t* c, int64_t M,
                                 int64_t N, int64_t K, int64_t ldc, void* workspace,
                                 int64_t workspace_bytes, void* stream) {
  int rc = check_gemm_shape(a, b, c, M, N, K, ldc);
  if (!rc) rc = check_workspace(workspace, workspace_bytes);
  if (rc) return rc;
  if (M == 0 || N == 0) return MXQ_OK;
  GemmArgs g{};
  g.a = a; g.b = b; g.d = c; g.M = M; g.N = N; g.K = K; g.ldd = ldc;
  return launch_gemm<kEpiI32, 0>(g, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int mxq_int8_gemm_dequant(const int8_t* a, const int8_t* b, const float* xs,
                                     const float* ws, int64_t ws_numel, const void* bias, void* d,
                                     int64_t M, int64_t N, int64_t K, int64_t ldd, int out_dtype,
                                     void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = check_gemm_shape(a, b, d, M, N, K, ldd);
  if (!rc) rc = check_workspace(workspace, workspace_bytes);
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
    case MXQ_DTYPE_F32: return launch_gemm<kEpiDequant, 0>(g, workspace, workspace_bytes, st);
    case MXQ_DTYPE_F16: return launch_gemm<kEpiDequant, 1>(g, workspace, workspace_bytes, st);
    case MXQ_DTYPE_BF16: return launch_gemm<kEpiDequant, 2>(g, workspace, workspace_bytes, st);
    default: return mxq_set_error(MXQ_ERR_UNSUPPORTED, "output dtype code %d", out_dtype);
  }
}

extern "C" int mxq_int8_gemm_dequant_gelu_absmax(const int8_t* a, const int8_t* b, const float* xs,
                                                 const float* ws, int64_t ws_numel,
                                                 const void* bias_bf16, void* h_bf16,
                                                 float* row_absmax, int64_t M, int64_t N,
                                                 int64_t K, int64_t ldh, void* workspace,
                                                 int64_t workspace_bytes, void* stream) {
  int rc = check_gemm_shape(a, b, h_bf16, M, N, K, ldh);
  if (!rc) rc = check_workspace(workspace, workspace_bytes);
  if (rc) return rc;
  if (M == 0 || N == 0) return MXQ_OK;
  if (!xs || !ws || !row_absmax) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  if (ws_numel != 1 && ws_numel != N) return mxq_set_error(MXQ_ERR_INVALID, "bad weight scale length");
  GemmArgs g{};
  g.a = a; g.b = b; g.xs = xs; g.ws = ws; g.bias = bias_bf16; g.d = h_bf16; g.row_absmax = row_absmax;
  g.M = M; g.N = N; g.K = K; g.ldd = ldh; g.ws_per_channel = ws_numel == N && N != 1;
  return launch_gemm<kEpiGelu, 2>(g, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int mxq_int8_gemm_dequant_swiglu(const int8_t* a, const int8_t* b, const float* xs,
                                            const float* ws, int64_t ws_numel, const void* bias_bf16,
                                            void* h_bf16, int64_t M, int64_t N, int64_t K, int64_t ldh,
                                            void* workspace, int64_t workspace_bytes, void* stream) {
  if (N % 32) return mxq_set_error(MXQ_ERR_INVALID, "SwiGLU fc1 width %lld must be a multiple of 32", (long long)N);
  int rc = check_gemm_shape(a, b, h_bf16, M, N / 2, K, ldh);
  if (!rc) rc = check_workspace(workspace, workspace_bytes);
  if (rc) return rc;
  if (M == 0 || N == 0) return MXQ_OK;
  if (!xs || !ws) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  if (ws_numel != 1 && ws_numel != N) return mxq_set_error(MXQ_ERR_INVALID, "bad weight scale length");
  GemmArgs g{};
  g.a = a; g.b = b; g.xs = xs; g.ws = ws; g.bias = bias_bf16; g.d = h_bf16;
  g.M = M; g.N = N; g.K = K; g.ldd = ldh; g.ws_per_channel = ws_numel == N && N != 1;
  return launch_gemm<kEpiSwiGLU, 2>(g, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int mxq_int8_gemm_gated_residual(const int8_t* a, const int8_t* b, const float* xs,
                                            const float* ws, int64_t ws_numel, const void* bias_bf16,
                                            void* residual_bf16, int64_t ldr, const void* gate_bf16,
                                            int64_t ldg, int64_t gate_count, const int32_t* gate_rows,
                                            int64_t M, int64_t N, int64_t K, void* workspace,
                                            int64_t workspace_bytes, void* stream) {
  int rc = check_gemm_shape(a, b, residual_bf16, M, N, K, ldr);
  if (!rc) rc = check_workspace(workspace, workspace_bytes);
  if (rc) return rc;
  if (M == 0 || N == 0) return MXQ_OK;
  if (!xs || !ws || !gate_bf16 || !gate_rows) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  if (ws_numel != 1 && ws_numel != N) return mxq_set_error(MXQ_ERR_INVALID, "bad weight scale length");
  if (ldg < N) return mxq_set_error(MXQ_ERR_INVALID, "gate stride %lld < N %lld", (long long)ldg, (long long)N);
  if (gate_count < 1) return mxq_set_error(MXQ_ERR_INVALID, "gate has no rows");
  GemmArgs g{};
  g.a = a; g.b = b; g.xs = xs; g.ws = ws; g.bias = bias_bf16; g.d = residual_bf16;
  g.res = (uint16_t*)residual_bf16; g.ldr = ldr; g.gate = (const uint16_t*)gate_bf16; g.ldg = ldg;
  g.gate_rows = gate_rows; g.gate_count = gate_count;
  g.M = M; g.N = N; g.K = K; g.ldd = ldr; g.ws_per_channel = ws_numel == N && N != 1;
  return launch_gemm<kEpiGatedRes, 2>(g, workspace, workspace_bytes, (hipStream_t)stream);
}
