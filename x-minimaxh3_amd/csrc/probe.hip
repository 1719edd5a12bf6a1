// MFMA ceiling probe: sustained v_mfma_i32_32x32x32_i8 throughput on given int8 operands with
// registers only (no memory traffic in the timed loop), and the shader clock it runs at.
//
// On MI355X the matrix cores' power draw depends on the operand bits: with constant operands the
// loop runs near the nominal clock, with random int8 operands the board power limit lowers the
// clock. A GEMM on the same data cannot beat this loop, so it is the measured roofline peak for
// that data (the nominal 5.0 POPS assumes 2.4 GHz).

#include "mxq_common.h"

namespace mxq {

// Each lane holds four A and two B fragments read from the operand buffers and cycles through
// them, so consecutive MFMAs see different operands as in a GEMM; eight independent
// accumulators keep the matrix pipe busy.
__global__ __launch_bounds__(256) void mfma_probe_kernel(const int8_t* __restrict__ a, int64_t a_chunks,
                                                         const int8_t* __restrict__ b, int64_t b_chunks,
                                                         int32_t* __restrict__ sink,
                                                         uint64_t* __restrict__ clocks, int iters) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  v4i fa[4], fb[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) fa[i] = reinterpret_cast<const v4i*>(a)[(t * 4 + i) % a_chunks];
#pragma unroll
  for (int i = 0; i < 2; ++i) fb[i] = reinterpret_cast<const v4i*>(b)[(t * 2 + i) % b_chunks];
  v16i acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = v16i{};
  const uint64_t c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i & 3], fb[i >> 2], acc[i], 0, 0, 0);
  }
  const uint64_t c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  int32_t s = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[i][r];
  sink[t] = s;
  if (threadIdx.x == 0) {
    clocks[blockIdx.x * 2 + 0] = c1 - c0;
    clocks[blockIdx.x * 2 + 1] = r1 - r0;
  }
}

// One wave64: the lane pairings of the DPP wave reductions. xor4[i] = lane_xor4(i); row16[i] =
// row16_sum_f64 of in[]; wsum[i] = wave_sum of float(in[]).
__global__ __launch_bounds__(64) void lane_exchange_kernel(const double* __restrict__ in, uint32_t* __restrict__ xor4,
                                                           double* __restrict__ row16, float* __restrict__ wsum) {
  const int i = threadIdx.x;
  xor4[i] = lane_xor4((uint32_t)i);
  row16[i] = row16_sum_f64(in[i]);
  wsum[i] = wave_sum((float)in[i]);
}

}  // namespace mxq

using namespace mxq;

extern "C" int mxq_probe_lane_exchange(const double* in, uint32_t* xor4, double* row16, float* wsum, void* stream) {
  if (!in || !xor4 || !row16 || !wsum) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  lane_exchange_kernel<<<1, 64, 0, (hipStream_t)stream>>>(in, xor4, row16, wsum);
  return mxq_check_launch("lane_exchange_kernel");
}

extern "C" int mxq_probe_mfma_i8(const int8_t* a, int64_t a_bytes, const int8_t* b, int64_t b_bytes,
                                 int32_t* sink, uint64_t* clocks, int64_t workgroups, int64_t iters,
                                 void* stream) {
  if (!a || !b || !sink || !clocks) return mxq_set_error(MXQ_ERR_INVALID, "null pointer");
  if (a_bytes < 16 || b_bytes < 16) return mxq_set_error(MXQ_ERR_INVALID, "operand buffers need at least 16 bytes");
  if ((uintptr_t)a % 16 || (uintptr_t)b % 16) return mxq_set_error(MXQ_ERR_INVALID, "operands must be 16-byte aligned");
  if (workgroups < 1 || workgroups > 65536 || iters < 1 || iters > (1 << 24))
    return mxq_set_error(MXQ_ERR_INVALID, "workgroups must be in [1, 65536] and iters in [1, 2^24]");
  mfma_probe_kernel<<<(unsigned)workgroups, 256, 0, (hipStream_t)stream>>>(a, a_bytes / 16, b, b_bytes / 16, sink,
                                                                          clocks, (int)iters);
  return mxq_check_launch("mfma_probe_kernel");
}
