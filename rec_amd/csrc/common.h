// Shared device helpers for the gfx950 quantized-KV attention kernels.
//
// Cache layout per layer, in 32-token blocks (bh = b * Hkv + h, C = capacity,
// a multiple of 32, blk = t / 32, t' = t % 32, p = pi(t') the position of
// token t' inside its block, see block_pos()):
//   int8 K codes   int8  [B][Hkv][C/32][2][32][64]   half m holds dims 64m..64m+63 of token t'
//   int4 K codes   uint8 [B][Hkv][C/32][32][4][2][8] row t', [byte run r][half m][8 bytes]: byte
//                                                   8r+i of half m = dims 64m+16r+2i, +1 (low nibble even)
//   int8 V codes   int8  [B][Hkv][C/32][128][32]     dim-major, token t' at position p
//   int4 V codes   uint8 [B][Hkv][C/32][2][16][4][4][4]  dim 16n+c, position p = 8g+e at
//                                                   [n/4][c][g][n%4][e/2], low nibble = even e
//   int8 scales    fp16  [B][Hkv][C/32][32]          one per (token, head), K and V, position p
//   int4 scale/zp  fp16  [B][Hkv][C/32][4][32]       per 32-dim group, slot s4_slot(p)
// Every load of the decode kernel reads one contiguous span: an int8 Q·Kᵀ
// operand is 16 tokens x 64 bytes of one K half, an int8 P·V operand 16 dims x
// 32 tokens, an int4 lane's K bytes (both halves) and V bytes (four dim
// blocks) are 16 adjacent bytes, and int4 scales / zero-points are read one
// dword per lane and handed out through LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rec {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef short v8s __attribute__((ext_vector_type(8)));

constexpr int HEAD_DIM = 128;
// Cache formats (kernel template arguments): 8 = int8 symmetric, 4 = uint4
// asymmetric group 32, FMT_A8 / FMT_A4 = MLX-style affine group 64 with bf16
// scale and bias (8-bit keys / 4-bit values), FMT_A8H / FMT_A4H the same with
// fp16 scale and bias (the keys' dtype of an fp16 model).
constexpr int FMT_A8 = 18;
constexpr int FMT_A4 = 14;
constexpr int FMT_A8H = 19;
constexpr int FMT_A4H = 15;
__host__ __device__ constexpr bool is_a8(int f) { return f == FMT_A8 || f == FMT_A8H; }
__host__ __device__ constexpr bool is_a4(int f) { return f == FMT_A4 || f == FMT_A4H; }
__host__ __device__ constexpr bool is_affine(int f) { return is_a8(f) || is_a4(f); }
__host__ __device__ constexpr bool meta_f16(int f) { return f == FMT_A8H || f == FMT_A4H; }
constexpr int FMT_BF = 16;  // bf16 K/V tensors (the KVStorage cache), prefill only
constexpr int GROUP_A = 64;
constexpr int BLOCK_T = 32;      // tokens per cache block and per wave iteration
constexpr int GROUP4 = 32;       // int4 group size along head_dim
constexpr float LOG2E = 1.4426950408889634f;
constexpr float NEG_INF = -__builtin_huge_valf();

enum InDtype { DT_F16 = 0, DT_BF16 = 1, DT_F32 = 2 };

// Position of token t (0..31) inside its 32-token block.  The Q·Kᵀ MFMA
// leaves lane group kg (0..3) holding the scores of tokens 16j + 4kg + i
// (j = 0..1, i = 0..3); storing those eight at positions 8kg .. 8kg+7 lets the
// lane read its V codes and scales with one load each.  Tokens t and t^1 stay
// neighbours (positions p and p^1), so a uint4 byte never straddles blocks.
__host__ __device__ constexpr int block_pos(int t) { return ((t >> 2) & 3) * 8 + (t >> 4) * 4 + (t & 3); }

// Slot of block position p in a 4-bit scale / zero-point row.  Inside each run
// of 8 positions the slots hold positions 0,4,1,5,2,6,3,7: a uint4 V nibble
// unpack yields the codes of positions (e, e+4) as one fp16 pair, and their
// scales (zero-points) then sit in one dword.
__host__ __device__ constexpr int s4_slot(int p) { return (p & ~7) | (2 * (p & 3)) | ((p >> 2) & 1); }

__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
  return (float)h;
}

__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
  _Float16 h = (_Float16)f;  // v_cvt_f16_f32, round-to-nearest-even
  return __builtin_bit_cast(uint16_t, h);
}

// Affine scale / bias words: two 16-bit values per dword, bf16 or (F16) fp16.
template <bool F16>
__device__ __forceinline__ float meta_lo(uint32_t w) {
  if constexpr (F16) return half_bits_to_float(w & 0xffffu);
  return __builtin_bit_cast(float, w << 16);
}
template <bool F16>
__device__ __forceinline__ float meta_hi(uint32_t w) {
  if constexpr (F16) return half_bits_to_float(w >> 16);
  return __builtin_bit_cast(float, w & 0xffff0000u);
}
template <bool F16>
__device__ __forceinline__ float meta_bits(uint32_t bits16) {
  if constexpr (F16) return half_bits_to_float(bits16);
  return __builtin_bit_cast(float, bits16 << 16);
}

// Load element i of a half/bfloat16/float array as float (exact).
__device__ __forceinline__ float load_as_float(const void* p, int64_t i, int dt) {
  if (dt == DT_F16) {
    return (float)((const _Float16*)p)[i];
  } else if (dt == DT_BF16) {
    uint32_t b = ((const uint16_t*)p)[i];
    return __builtin_bit_cast(float, b << 16);
  }
  return ((const float*)p)[i];
}

// Store consecutive output elements i, i+1 (, i+2, i+3) of an fp32, bf16 or
// fp16 array (dt a DT_* code); 16-bit outputs are rounded to nearest even by
// the hardware conversions, as a cast of the fp32 result would round them.
__device__ __forceinline__ void store_out2(void* out, int64_t i, v2f o, int dt) {
  if (dt == DT_F32) {
    *(v2f*)((float*)out + i) = o;
  } else if (dt == DT_BF16) {
    const __bf16 a = (__bf16)o[0], b = (__bf16)o[1];
    *(uint32_t*)((uint16_t*)out + i) =
        (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
  } else {
    const _Float16 a = (_Float16)o[0], b = (_Float16)o[1];
    *(uint32_t*)((uint16_t*)out + i) =
        (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
  }
}
__device__ __forceinline__ void store_out4(void* out, int64_t i, v4f o, int dt) {
  if (dt == DT_F32) {
    *(v4f*)((float*)out + i) = o;
  } else {
    store_out2(out, i, (v2f){o[0], o[1]}, dt);
    store_out2(out, i + 2, (v2f){o[2], o[3]}, dt);
  }
}

// fp16 round-to-nearest-even of a non-negative float, saturating at 65504.
// float -> bf16 bits, round to nearest even (finite inputs).
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ uint16_t half_bits_saturate(float f) {
  uint16_t b = float_to_half_bits(f);
  if ((b & 0x7fff) == 0x7c00) b = (b & 0x8000) | 0x7bff;
  return b;
}

// Exchange with the lane 8 positions away inside each row of 16 (DPP row_ror:8).
__device__ __forceinline__ int dpp_ror8(int x) {
  return __builtin_amdgcn_mov_dpp(x, 0x128, 0xf, 0xf, false);
}
__device__ __forceinline__ float dpp_ror8f(float x) {
  return __builtin_bit_cast(float, dpp_ror8(__builtin_bit_cast(int, x)));
}

// (x & m) | o in one v_and_or_b32 (the compiler splits it when both constants
// would need the single scalar operand slot).
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t o) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(m), "v"(o));
  return r;
}

// Online softmax: the running max (log2 units) is moved only when a score
// exceeds it by more than this, so probabilities stay below 2^8 — as exact in
// fp16 / bf16 operands and fp32 sums as ones below 1 — and the rescale of the
// accumulators runs rarely.
constexpr float RESCALE_GAP = 8.f;

// ---- cross-lane combines without LDS round trips ----
// DPP moves inside rows of 16 lanes; v_permlane16_swap / v_permlane32_swap
// (gfx950) across rows and halves.  A swap of x with itself returns
// {x[l & ~m], x[l | m]} (m = 16 or 32), so combining the pair gives every lane
// the xor-m butterfly of x, the same value in both partners.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
constexpr int DPP_XOR1 = 0xb1;         // quad_perm [1, 0, 3, 2]
constexpr int DPP_XOR2 = 0x4e;         // quad_perm [2, 3, 0, 1]
constexpr int DPP_HALF_MIRROR = 0x141;  // lane i <-> 7 - i in each 8
constexpr int DPP_MIRROR = 0x140;       // lane i <-> 15 - i in each 16
constexpr int DPP_ROR8 = 0x128;         // lane i <-> i ^ 8 in each 16

__device__ __forceinline__ void pair16(float x, float& lo, float& hi) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const uint32_t a = r[0], b = r[1];  // copies: a bit_cast of a vector subscript reads element 0
  lo = __builtin_bit_cast(float, a);
  hi = __builtin_bit_cast(float, b);
}
__device__ __forceinline__ void pair32(float x, float& lo, float& hi) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const uint32_t a = r[0], b = r[1];
  lo = __builtin_bit_cast(float, a);
  hi = __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float sum_xor16(float x) {
  float a, b;
  pair16(x, a, b);
  return a + b;
}
__device__ __forceinline__ float sum_xor32(float x) {
  float a, b;
  pair32(x, a, b);
  return a + b;
}
// Maximum that propagates NaN (v_maximum3_f32 on gfx950).  fmaxf must quiet a
// signaling NaN input, so the compiler puts a v_max_f32 x, x, x in front of
// every operand it cannot prove canonical (matrix-core results among them);
// this one needs none, and a chain of n operands costs ceil((n - 1) / 2)
// instructions.
__device__ __forceinline__ float maxp(float a, float b) { return __builtin_elementwise_maximum(a, b); }

__device__ __forceinline__ float max_xor16(float x) {
  float a, b;
  pair16(x, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float max_xor32(float x) {
  float a, b;
  pair32(x, a, b);
  return fmaxf(a, b);
}

template <int CTRL>
__device__ __forceinline__ int dpp_i(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xf, 0xf, false);
}

// max / min / sum over each group of 8 or 16 lanes (every lane receiving its
// group's result), and over the 64 lanes
__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp_f<DPP_XOR1>(x));
  x = fmaxf(x, dpp_f<DPP_XOR2>(x));
  x = fmaxf(x, dpp_f<DPP_HALF_MIRROR>(x));
  return fmaxf(x, dpp_f<DPP_MIRROR>(x));
}
__device__ __forceinline__ float row16_min(float x) {
  x = fminf(x, dpp_f<DPP_XOR1>(x));
  x = fminf(x, dpp_f<DPP_XOR2>(x));
  x = fminf(x, dpp_f<DPP_HALF_MIRROR>(x));
  return fminf(x, dpp_f<DPP_MIRROR>(x));
}
__device__ __forceinline__ int group8_sum(int x) {
  x += dpp_i<DPP_XOR1>(x);
  x += dpp_i<DPP_XOR2>(x);
  return x + dpp_i<DPP_HALF_MIRROR>(x);
}
__device__ __forceinline__ float group8_sum(float x) {
  x += dpp_f<DPP_XOR1>(x);
  x += dpp_f<DPP_XOR2>(x);
  return x + dpp_f<DPP_HALF_MIRROR>(x);
}
__device__ __forceinline__ float wave_max(float x) { return max_xor32(max_xor16(row16_max(x))); }
__device__ __forceinline__ float wave_sum(float x) {
  x = group8_sum(x);
  x += dpp_f<DPP_MIRROR>(x);
  return sum_xor32(sum_xor16(x));
}

// Four signed int8 codes -> two packed fp16 pairs, exactly.
// The code is biased to unsigned (xor 0x80), glued under the fp16 exponent of
// 1024 with v_perm, then 1024 + 128 is subtracted: (1024 + 128 + q) - 1152 = q.
__device__ __forceinline__ void i8x4_to_h2x2(uint32_t w, v2h& lo, v2h& hi) {
  const uint32_t u = w ^ 0x80808080u;
  const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
  const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
  const v2h bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  lo = __builtin_bit_cast(v2h, a) + bias;
  hi = __builtin_bit_cast(v2h, b) + bias;
}

// Eight int8 codes in two dwords -> eight fp16 values in order.
__device__ __forceinline__ v8h i8x8_to_h8(uint32_t w0, uint32_t w1) {
  v2h a, b, c, d;
  i8x4_to_h2x2(w0, a, b);
  i8x4_to_h2x2(w1, c, d);
  v8h r;
  r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
  r[4] = c[0]; r[5] = c[1]; r[6] = d[0]; r[7] = d[1];
  return r;
}

// Eight uint4 codes in one dword (byte j = elements 2j | 2j+1 << 4) -> eight
// fp16 values in the order [e0, e4, e1, e5, e2, e6, e3, e7].
__device__ __forceinline__ v8h u4x8_to_h8_interleaved(uint32_t w) {
  const v2h bias = {(_Float16)-1024.0f, (_Float16)-1024.0f};
  v8h r;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    uint32_t t = ((w >> (4 * s)) & 0x000f000fu) | 0x64006400u;
    v2h h = __builtin_bit_cast(v2h, t) + bias;
    r[2 * s] = h[0];
    r[2 * s + 1] = h[1];
  }
  return r;
}

// ---- raw buffer loads ----------------------------------------------------
// A buffer resource bounds every load: offsets past its records read zero
// without touching memory, so loads of absent data are issued unconditionally.
constexpr int BUF_NT = 2;  // cache policy: nontemporal (the KV is streamed once)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, int64_t bytes) {
  // gfx9 buffer descriptor word 3 for raw (stride 0) dword access
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ float half_at(const v4i& w, int idx) {
  const uint32_t x = (uint32_t)w[idx >> 1];
  return half_bits_to_float((idx & 1) ? (x >> 16) : (x & 0xffff));
}

// The builtins return unsigned vectors; convert with bit_cast only (an
// implicit conversion to a signed vector type can turn into a splat of lane 0).
template <int POL = BUF_NT>
__device__ __forceinline__ v4i ld128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, POL));
}
template <int POL = BUF_NT>
__device__ __forceinline__ v2i ld64(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, POL));
}
template <int POL = BUF_NT>
__device__ __forceinline__ uint32_t ld32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, POL);
}

// Ordering of LDS accesses between the lanes of one wavefront (no hardware
// barrier: a wavefront's LDS operations execute in order).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace rec
