// Shared pieces of the group-scaled W4A8 kernels (w4a8.hip, w4a8_g128.hip).
#pragma once

#include "mxq_common.h"

namespace mxq {

constexpr int kW4BK = 128;

struct W4Args {
  const int8_t* a;
  const float* xs;
  const uint8_t* w;       // [N, K/2]
  const uint16_t* gs;     // [K/G, N] fp16
  const void* bias;
  void* d;
  int64_t M, N, K, ldd;
  int group_tiles;        // K-stages per group (G / 128)
  int tiles_m, tiles_n;
};

// 4 packed bytes (8 codes, even k low nibble) -> 8 int8 holding 16 (c - 8), natural k order.
MXQ_DEVICE void unpack8(uint32_t w, uint32_t& o0, uint32_t& o1) {
  const uint32_t x = w ^ 0x88888888u;
  const uint32_t xs = x << 4;
  o0 = __builtin_amdgcn_perm(x, xs, 0x05010400u) & 0xF0F0F0F0u;
  o1 = __builtin_amdgcn_perm(x, xs, 0x07030602u) & 0xF0F0F0F0u;
}

// The prepared layout (mxq_w4a8_prepare_grouped): each 32-bit word of a weight row still holds
// the 8 codes of k = 8w .. 8w + 7, but byte j holds (c[8w + j] ^ 8) in its low nibble and
// (c[8w + 4 + j] ^ 8) in its high nibble -- the offset-8 code as a 4-bit two's complement value
// c - 8. Unpacking to 16 (c - 8) per int8 in natural k order is then a shift and two masks.
MXQ_DEVICE void unpack8_prepared(uint32_t w, uint32_t& o0, uint32_t& o1) {
  o0 = (w << 4) & 0xF0F0F0F0u;
  o1 = w & 0xF0F0F0F0u;
}

// The group-128 pipelined kernel (w4a8_g128.hip): needs group size 128, N % 8 == 0 and 16-byte
// aligned scale rows; `prepared` selects the weight layout. Returns MXQ_ERR_UNSUPPORTED without
// launching (and without setting an error) when the operands are too large for its 32-bit
// offsets.
int launch_w4_g128(W4Args p, int out_dtype, bool prepared, hipStream_t st);

}  // namespace mxq
