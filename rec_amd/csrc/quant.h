// Quantize-on-append: one wavefront turns one (b, h, t) row of 128 values into
// cache codes and scales.  Restates the append step of
// engine/src/rec_mlx/model.py:77-81 (quantize the new rows, write them at
// [prev:offset]) for this library's int8 / uint4 formats.  The arithmetic is
// IEEE float32 (correctly rounded divide, round-half-even rint, fp16 RNE) so
// codes and scales are bit-identical to the CPU restatement.
#pragma once

#include "common.h"

namespace rec {

struct RowSrc {
  const void* p;
  int dtype;
  int64_t sb, sh, st;  // element strides for batch, head, token (dim stride 1)
};

__device__ __forceinline__ int64_t row_base(const RowSrc& s, int b, int h, int t) {
  return (int64_t)b * s.sb + (int64_t)h * s.sh + (int64_t)t * s.st;
}

// int8 symmetric, one fp16 scale per row.  Lane l owns dims 2l, 2l+1.
// Returns the two codes; the caller stores them in its layout.
__device__ __forceinline__ void quantize_i8_pair(float x0, float x1, int& q0, int& q1, uint16_t& sbits) {
  float amax = wave_max(fmaxf(fabsf(x0), fabsf(x1)));
  sbits = half_bits_saturate(amax / 127.0f);
  const float s = half_bits_to_float(sbits);
  q0 = 0;
  q1 = 0;
  if (s != 0.0f) {
    q0 = (int)fminf(fmaxf(__builtin_rintf(x0 / s), -127.0f), 127.0f);
    q1 = (int)fminf(fmaxf(__builtin_rintf(x1 / s), -127.0f), 127.0f);
  }
}

// uint4 asymmetric per 32-dim group (16 lanes).  Lane l owns dims 2l, 2l+1.
__device__ __forceinline__ void quantize_u4_pair(float x0, float x1, int& q0, int& q1, uint16_t& sbits,
                                                 uint16_t& zbits) {
  float mn = fminf(x0, x1), mx = fmaxf(x0, x1);
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) {
    mn = fminf(mn, __shfl_xor(mn, m, 64));
    mx = fmaxf(mx, __shfl_xor(mx, m, 64));
  }
  mn = fminf(mn, 0.0f);
  mx = fmaxf(mx, 0.0f);
  sbits = half_bits_saturate((mx - mn) / 15.0f);
  const float s = half_bits_to_float(sbits);
  q0 = 0;
  q1 = 0;
  float z = 0.0f;
  if (s != 0.0f) {
    z = fminf(fmaxf(__builtin_rintf(-mn / s), 0.0f), 15.0f) + 0.0f;  // +0, never -0
    q0 = (int)fminf(fmaxf(__builtin_rintf(x0 / s) + z, 0.0f), 15.0f);
    q1 = (int)fminf(fmaxf(__builtin_rintf(x1 / s) + z, 0.0f), 15.0f);
  }
  zbits = float_to_half_bits(z);
}

// Cache addressing (element offsets), see the layout table in common.h.
__device__ __forceinline__ int64_t i8_row_off(int64_t bh, int64_t cap, int64_t t) { return (bh * cap + t) * HEAD_DIM; }
__device__ __forceinline__ int64_t i8_blk_off(int64_t bh, int64_t cap, int64_t t, int d) {
  return bh * cap * HEAD_DIM + (t >> 6) * (BLOCK_T * HEAD_DIM) + (int64_t)d * BLOCK_T + (t & 63);
}
__device__ __forceinline__ int64_t u4_row_off(int64_t bh, int64_t cap, int64_t t) { return (bh * cap + t) * (HEAD_DIM / 2); }
__device__ __forceinline__ int64_t u4_blk_byte(int64_t bh, int64_t cap, int64_t t, int d) {
  return bh * cap * (HEAD_DIM / 2) + (t >> 6) * (BLOCK_T * HEAD_DIM / 2) + (int64_t)d * (BLOCK_T / 2) + ((t & 63) >> 1);
}
__device__ __forceinline__ int64_t u4_scale_off(int64_t bh, int64_t cap, int64_t t, int g) {
  return bh * cap * 4 + (t >> 6) * (4 * BLOCK_T) + g * BLOCK_T + (t & 63);
}

// Quantize row (b, h, t_src) of `src` and store it at cache position `pos`.
// kind 0 = K (row-major codes), kind 1 = V (token-blocked codes).  uint4 V
// rows share bytes with their neighbour, so they go through append_v4_pair.
template <int BITS>
__device__ __forceinline__ void append_row(const RowSrc& src, int b, int h, int t_src, int kind, void* codes,
                                           uint16_t* scales, uint16_t* zeros, int64_t bh, int64_t cap,
                                           int64_t pos, int lane) {
  const int64_t base = row_base(src, b, h, t_src);
  const float x0 = load_as_float(src.p, base + 2 * lane, src.dtype);
  const float x1 = load_as_float(src.p, base + 2 * lane + 1, src.dtype);
  if constexpr (BITS == 8) {
    int q0, q1;
    uint16_t sb;
    quantize_i8_pair(x0, x1, q0, q1, sb);
    int8_t* c = (int8_t*)codes;
    if (kind == 0) {
      uint16_t packed = (uint16_t)((q0 & 0xff) | ((q1 & 0xff) << 8));
      ((uint16_t*)(c + i8_row_off(bh, cap, pos)))[lane] = packed;
    } else {
      c[i8_blk_off(bh, cap, pos, 2 * lane)] = (int8_t)q0;
      c[i8_blk_off(bh, cap, pos, 2 * lane + 1)] = (int8_t)q1;
    }
    if (lane == 0) scales[bh * cap + pos] = sb;
  } else {
    int q0, q1;
    uint16_t sb, zb;
    quantize_u4_pair(x0, x1, q0, q1, sb, zb);
    ((uint8_t*)codes)[u4_row_off(bh, cap, pos) + lane] = (uint8_t)(q0 | (q1 << 4));
    if ((lane & 15) == 0) {
      const int g = lane >> 4;
      scales[u4_scale_off(bh, cap, pos, g)] = sb;
      zeros[u4_scale_off(bh, cap, pos, g)] = zb;
    }
  }
}

// uint4 V: the byte pair of cache positions (2p, 2p+1).  Rows whose flag is
// false keep the nibble already in the cache; each byte is written once.
__device__ __forceinline__ void append_v4_pair(const RowSrc& src, int b, int h, int t_even, bool has_even,
                                               bool has_odd, uint8_t* codes, uint16_t* scales, uint16_t* zeros,
                                               int64_t bh, int64_t cap, int64_t pos_even, int lane) {
  int qe0 = 0, qe1 = 0, qo0 = 0, qo1 = 0;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const bool has = r == 0 ? has_even : has_odd;
    if (!has) continue;  // wave-uniform
    const int64_t base = row_base(src, b, h, t_even + r);
    const float x0 = load_as_float(src.p, base + 2 * lane, src.dtype);
    const float x1 = load_as_float(src.p, base + 2 * lane + 1, src.dtype);
    int q0, q1;
    uint16_t sb, zb;
    quantize_u4_pair(x0, x1, q0, q1, sb, zb);
    if (r == 0) { qe0 = q0; qe1 = q1; } else { qo0 = q0; qo1 = q1; }
    if ((lane & 15) == 0) {
      const int g = lane >> 4;
      scales[u4_scale_off(bh, cap, pos_even + r, g)] = sb;
      zeros[u4_scale_off(bh, cap, pos_even + r, g)] = zb;
    }
  }
  const int64_t a0 = u4_blk_byte(bh, cap, pos_even, 2 * lane);
  const int64_t a1 = u4_blk_byte(bh, cap, pos_even, 2 * lane + 1);
  uint8_t o0 = 0, o1 = 0;
  if (!(has_even && has_odd)) { o0 = codes[a0]; o1 = codes[a1]; }
  const int lo0 = has_even ? qe0 : (o0 & 15), hi0 = has_odd ? qo0 : (o0 >> 4);
  const int lo1 = has_even ? qe1 : (o1 & 15), hi1 = has_odd ? qo1 : (o1 >> 4);
  codes[a0] = (uint8_t)(lo0 | (hi0 << 4));
  codes[a1] = (uint8_t)(lo1 | (hi1 << 4));
}

}  // namespace rec
