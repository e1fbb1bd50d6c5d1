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
  int vec;             // p is 16-byte aligned and every stride a multiple of 4 elements
};

// Elements i, i+1 (i even) of a row as floats: one load when src.vec.
__device__ __forceinline__ void load2_as_float(const RowSrc& s, int64_t i, float& x0, float& x1) {
  if (s.vec) {
    if (s.dtype == DT_F32) {
      const v2f v = *(const v2f*)((const float*)s.p + i);
      x0 = v[0];
      x1 = v[1];
    } else {
      const uint32_t w = *(const uint32_t*)((const uint16_t*)s.p + i);
      if (s.dtype == DT_F16) {
        x0 = half_bits_to_float(w & 0xffffu);
        x1 = half_bits_to_float(w >> 16);
      } else {
        x0 = __builtin_bit_cast(float, w << 16);
        x1 = __builtin_bit_cast(float, w & 0xffff0000u);
      }
    }
  } else {
    x0 = load_as_float(s.p, i, s.dtype);
    x1 = load_as_float(s.p, i + 1, s.dtype);
  }
}

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
  float mn = row16_min(fminf(x0, x1)), mx = row16_max(fmaxf(x0, x1));
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

// MLX-style affine quantization of one group of 64 (32 lanes, 2 elements
// each; restates mx.quantize's affine_quantize, mlx 0.32.0): the range is
// [min w, max(0, max w)], the extreme of larger magnitude (the edge) is made
// exact by stretching the step, codes are round((w - bias) / scale) clamped to
// [0, 2^BITS - 1] (round = half away from zero), scale and bias are stored as
// bf16 (F16: fp16, the keys' dtype of an fp16 model), rounded to nearest even.
// Float32 arithmetic with correctly rounded division, so the codes and bits
// match the CPU restatement exactly.
template <int BITS, bool F16 = false>
__device__ __forceinline__ void quantize_affine_pair(float x0, float x1, int& q0, int& q1, uint16_t& sbits,
                                                     uint16_t& bbits) {
  constexpr float n_bins = (float)((1 << BITS) - 1);
  float a, b;
  float mn = row16_min(fminf(x0, x1)), mx = row16_max(fmaxf(x0, x1));
  pair16(mn, a, b);  // the two rows of the 32-lane group
  mn = fminf(a, b);
  mx = max_xor16(mx);
  mx = fmaxf(mx, 0.0f);
  float scale = fmaxf((mx - mn) / n_bins, 1e-7f);
  const bool side = fabsf(mn) > fabsf(mx);
  scale = side ? scale : -scale;
  const float edge = side ? mn : mx;
  const float qe = __builtin_roundf(edge / scale);
  const bool at_zero = qe == 0.0f;
  scale = at_zero ? scale : edge / qe;
  const float bias = at_zero ? 0.0f : edge;
  q0 = (int)fminf(fmaxf(__builtin_roundf((x0 - bias) / scale), 0.0f), n_bins);
  q1 = (int)fminf(fmaxf(__builtin_roundf((x1 - bias) / scale), 0.0f), n_bins);
  sbits = F16 ? float_to_half_bits(scale) : float_to_bf16_bits(scale);
  bbits = F16 ? float_to_half_bits(bias) : float_to_bf16_bits(bias);
}

// Cache addressing in elements (bytes for codes), see the layout table in common.h.
__device__ __forceinline__ int64_t blk_base(int64_t bh, int64_t cap, int64_t t, int block_elems) {
  return (bh * (cap / BLOCK_T) + (t >> 5)) * block_elems;
}
// int8 K: byte of dim d
__device__ __forceinline__ int64_t k8_off(int64_t bh, int64_t cap, int64_t t, int d) {
  return blk_base(bh, cap, t, 4096) + (d >> 6) * 2048 + (t & 31) * 64 + (d & 63);
}
// int4 K: byte holding dims d, d+1 (d even).  Row t of the block is 64 bytes:
// [4 dim-groups of 16 per half][half m][8 bytes], so the 16 bytes a lane reads
// (dims 16g..16g+15 of both halves) are contiguous.
__device__ __forceinline__ int64_t k4_off(int64_t bh, int64_t cap, int64_t t, int d) {
  const int b = (d & 63) >> 1;  // byte inside the half
  return blk_base(bh, cap, t, 2048) + (t & 31) * 64 + (b >> 3) * 16 + (d >> 6) * 8 + (b & 7);
}
// int8 V: byte of dim d.  For d = 16n + c and position p = 8kg + e the byte
// sits at [n/2][c][kg][n%2][e]: the 8 bytes of (d, kg) for n = 2h, 2h+1 are
// one 16-byte run, so a lane reads its 64 bytes with four 16-byte loads.
__device__ __forceinline__ int64_t v8_off(int64_t bh, int64_t cap, int64_t t, int d) {
  const int p = block_pos((int)(t & 31)), n = d >> 4, c = d & 15;
  return blk_base(bh, cap, t, 4096) + (n >> 1) * 1024 + (c * 4 + (p >> 3)) * 16 + (n & 1) * 8 + (p & 7);
}
// int4 V: byte holding token t (and its neighbour t^1) of dim d.  For dim
// d = 16n + c and position p = 8kg + e the byte sits at
// [n/4][c][kg][n%4][e/2]: the 4 bytes of (d, kg) for n = 4h..4h+3 are one
// 16-byte run, so a lane reads its 32 bytes with two 16-byte loads.
__device__ __forceinline__ int64_t v4_off(int64_t bh, int64_t cap, int64_t t, int d) {
  const int p = block_pos((int)(t & 31)), n = d >> 4, c = d & 15;
  return blk_base(bh, cap, t, 2048) + (n >> 2) * 1024 + (c * 4 + (p >> 3)) * 16 + (n & 3) * 4 + ((p & 7) >> 1);
}
// per-token scale (int8)
__device__ __forceinline__ int64_t s8_off(int64_t bh, int64_t cap, int64_t t) {
  return blk_base(bh, cap, t, 32) + block_pos((int)(t & 31));
}
// per-(token, group) scale / zero-point (int4), at slot s4_slot(position)
__device__ __forceinline__ int64_t s4_off(int64_t bh, int64_t cap, int64_t t, int g) {
  return blk_base(bh, cap, t, 128) + g * 32 + s4_slot(block_pos((int)(t & 31)));
}

// affine scale (which 0) or bias (which 1) of group g (0..1), at slot s4_slot(position)
__device__ __forceinline__ int64_t sa_off(int64_t bh, int64_t cap, int64_t t, int which, int g) {
  return blk_base(bh, cap, t, 128) + which * 64 + g * 32 + s4_slot(block_pos((int)(t & 31)));
}

// Quantize row (b, h, t_src) of `src` and store it at cache position `pos`.
// kind 0 = K (row-major codes), kind 1 = V (token-blocked codes).  uint4 V
// rows share bytes with their neighbour, so they go through append_v4_pair.
template <int BITS>
__device__ __forceinline__ void append_row(const RowSrc& src, int b, int h, int t_src, int kind, void* codes,
                                           uint16_t* scales, uint16_t* zeros, int64_t bh, int64_t cap,
                                           int64_t pos, int lane) {
  const int64_t base = row_base(src, b, h, t_src);
  float x0, x1;
  load2_as_float(src, base + 2 * lane, x0, x1);
  if constexpr (is_a8(BITS)) {  // affine 8-bit keys: uint8 codes in the int8 K layout
    int q0, q1;
    uint16_t sb, bb;
    quantize_affine_pair<8, meta_f16(BITS)>(x0, x1, q0, q1, sb, bb);
    *(uint16_t*)((uint8_t*)codes + k8_off(bh, cap, pos, 2 * lane)) = (uint16_t)(q0 | (q1 << 8));
    if ((lane & 31) == 0) {
      scales[sa_off(bh, cap, pos, 0, lane >> 5)] = sb;
      scales[sa_off(bh, cap, pos, 1, lane >> 5)] = bb;
    }
  } else if constexpr (BITS == 8) {
    int q0, q1;
    uint16_t sb;
    quantize_i8_pair(x0, x1, q0, q1, sb);
    int8_t* c = (int8_t*)codes;
    if (kind == 0) {
      *(uint16_t*)(c + k8_off(bh, cap, pos, 2 * lane)) = (uint16_t)((q0 & 0xff) | ((q1 & 0xff) << 8));
    } else {
      c[v8_off(bh, cap, pos, 2 * lane)] = (int8_t)q0;
      c[v8_off(bh, cap, pos, 2 * lane + 1)] = (int8_t)q1;
    }
    if (lane == 0) scales[s8_off(bh, cap, pos)] = sb;
  } else {
    int q0, q1;
    uint16_t sb, zb;
    quantize_u4_pair(x0, x1, q0, q1, sb, zb);
    ((uint8_t*)codes)[k4_off(bh, cap, pos, 2 * lane)] = (uint8_t)(q0 | (q1 << 4));
    if ((lane & 15) == 0) {
      const int g = lane >> 4;
      scales[s4_off(bh, cap, pos, g)] = sb;
      zeros[s4_off(bh, cap, pos, g)] = zb;
    }
  }
}

// uint4 V: the byte shared by tokens (2p, 2p+1) (block positions p', p'^1 with
// the even token in the low nibble).  Rows whose flag is false keep the nibble
// already in the cache; each byte is written once.
// AFFINE: MLX-style affine group 64 (scale and bias in `scales`, `zeros`
// unused), F16: stored as fp16 rather than bf16.
template <bool AFFINE = false, bool F16 = false>
__device__ __forceinline__ void append_v4_pair(const RowSrc& src, int b, int h, int t_even, bool has_even,
                                               bool has_odd, uint8_t* codes, uint16_t* scales, uint16_t* zeros,
                                               int64_t bh, int64_t cap, int64_t pos_even, int lane) {
  int qe0 = 0, qe1 = 0, qo0 = 0, qo1 = 0;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const bool has = r == 0 ? has_even : has_odd;
    if (!has) continue;  // wave-uniform
    const int64_t base = row_base(src, b, h, t_even + r);
    float x0, x1;
    load2_as_float(src, base + 2 * lane, x0, x1);
    int q0, q1;
    uint16_t sb, zb;
    if constexpr (AFFINE) {
      quantize_affine_pair<4, F16>(x0, x1, q0, q1, sb, zb);
      if ((lane & 31) == 0) {
        scales[sa_off(bh, cap, pos_even + r, 0, lane >> 5)] = sb;
        scales[sa_off(bh, cap, pos_even + r, 1, lane >> 5)] = zb;
      }
    } else {
      quantize_u4_pair(x0, x1, q0, q1, sb, zb);
      if ((lane & 15) == 0) {
        const int g = lane >> 4;
        scales[s4_off(bh, cap, pos_even + r, g)] = sb;
        zeros[s4_off(bh, cap, pos_even + r, g)] = zb;
      }
    }
    if (r == 0) { qe0 = q0; qe1 = q1; } else { qo0 = q0; qo1 = q1; }
  }
  const int64_t a0 = v4_off(bh, cap, pos_even, 2 * lane);
  const int64_t a1 = v4_off(bh, cap, pos_even, 2 * lane + 1);
  uint8_t o0 = 0, o1 = 0;
  if (!(has_even && has_odd)) { o0 = codes[a0]; o1 = codes[a1]; }
  const int lo0 = has_even ? qe0 : (o0 & 15), hi0 = has_odd ? qo0 : (o0 >> 4);
  const int lo1 = has_even ? qe1 : (o1 & 15), hi1 = has_odd ? qo1 : (o1 >> 4);
  codes[a0] = (uint8_t)(lo0 | (hi0 << 4));
  codes[a1] = (uint8_t)(lo1 | (hi1 << 4));
}

}  // namespace rec
