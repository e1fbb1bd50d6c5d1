// Chunked prefill of a few queries over the quantized caches (int8, uint4,
// mixed int8 / uint4 and affine): the
// decode's streaming structure with the chunk's (query, head) rows as matrix
// columns.
//
// Restates the same branch as prefill.hip (engine/src/rec_mlx/model.py:191-203:
// the L new tokens are cached first, then their queries attend over the whole
// cache with the causal mask of model.py:122-125 and the per-head sinks).
// For a short chunk -- a few draft tokens, a short turn -- the tiled prefill
// kernel spends each 128-token tile's conversion, LDS staging and barriers on
// 16-row tiles that are mostly empty; here, as in the decode, every wave
// streams its 32-token chunks from HBM into registers and the tile is never
// staged.  The (query, head) rows of one KV head, numbered query·G + head as
// in prefill.hip, fill NT column tiles of 16 (NT <= 4) per workgroup; more
// rows than one workgroup's 16·NT are split into row groups, one workgroup
// each (below):
//   * Q·Kᵀ on 16x16x32 bf16 (fp16 for fp16 queries) MFMAs: A = 16 tokens x 32
//     dims of the int8 K block converted in registers (exact), B = the rows'
//     query elements of the same dims (a lane holds dims 64m + 16kg + 8h ..
//     +7 for k-step 2m + h, the order the int8 block hands its bytes out);
//   * online softmax per column with the decode's lazy running max, the K
//     row scale and the softmax scale applied to the fp32 scores;
//   * P·V on 16x16x32 fp16 MFMAs: A = Vᵀ (int8 codes, exact in fp16), B =
//     P' = p·s (the token's V scale) as an fp16 high part and, when the first
//     query sees fewer than EXACT_PV_BELOW keys, its rounding remainder in a
//     second MFMA (as the tiled kernel does).
// The uint4 pair (4-bit K and V, fp16 scale and zero-point per 32 dims) and
// the affine pair (8-bit K, 4-bit V, group 64, bf16 or fp16 scale and bias) take the
// same loop with the values formed in registers as the tiled kernel forms
// them in LDS: K x̂ = q·s + b (affine) or (q − z)·s (uint4, q − z exact in
// fp16) in fp32, rounded once to the query dtype (the A operand), V x̂
// likewise, and P' = p.  Under fp16 queries P·V is the fp16
// product as above; under bf16 queries the bf16 V value enters a bf16 MFMA
// as it is, with P split into bf16 high and low parts.
// Work decomposition: one workgroup per (key split, KV head, row group) and
// batch row, with the prefill's split plan (128-token aligned ranges); 4
// waves take 32-token chunks in turn from a 2-deep ring of loads.  The row
// groups of one (split, KV head) read the same K/V bytes, so their
// workgroups are numbered 8 apart: workgroup i runs on XCD i % 8, and the
// groups run there at about the same time, all but the first finding the
// bytes in that XCD's L2 (20 queries x 8 heads over 32K keys, int8: 36.4 ->
// 32.0 us against the tiled kernel).  Each workgroup merges its waves in LDS
// and writes the normalised output (one split) or its unnormalised partial
// in the prefill workspace layout, which prefill_merge_kernel combines.
#include "kernels.h"

namespace rec {
namespace {

constexpr int FW = 4;        // wavefronts per workgroup
constexpr int FCH = 32;      // tokens per chunk (one cache block)
constexpr int FPR = HEAD_DIM + 4;  // LDS row pitch of a wave partial (floats)
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

template <bool BF16>
struct FewT;
template <>
struct FewT<true> {
  typedef v8bf vec;
  static __device__ __forceinline__ v4f mfma(vec a, vec b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  // eight int8 codes (two dwords) -> bf16, exactly
  static __device__ __forceinline__ vec codes(uint32_t w0, uint32_t w1) {
    vec r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      r[e] = (__bf16)(float)(int8_t)(w0 >> (8 * e));
      r[4 + e] = (__bf16)(float)(int8_t)(w1 >> (8 * e));
    }
    return r;
  }
  static __device__ __forceinline__ __bf16 from_float(float x) { return (__bf16)x; }  // nearest even
  // a dequantized V value as the reference holds it (bf16), widened to fp16
  static __device__ __forceinline__ _Float16 v_elem(float x) { return (_Float16)(float)(__bf16)x; }
};
template <>
struct FewT<false> {
  typedef v8h vec;
  static __device__ __forceinline__ v4f mfma(vec a, vec b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ vec codes(uint32_t w0, uint32_t w1) { return i8x8_to_h8(w0, w1); }
  static __device__ __forceinline__ _Float16 from_float(float x) { return (_Float16)x; }
  static __device__ __forceinline__ _Float16 v_elem(float x) { return (_Float16)x; }
};

// eight affine 8-bit K codes (two dwords, unsigned) -> x̂ = q·s + b in the
// query dtype, one fp32 fma and one rounding each
template <bool BF16>
__device__ __forceinline__ typename FewT<BF16>::vec affine8(uint32_t w0, uint32_t w1, float s, float b) {
  typename FewT<BF16>::vec r;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    r[e] = FewT<BF16>::from_float(__builtin_fmaf((float)((w0 >> (8 * e)) & 0xffu), s, b));
    r[4 + e] = FewT<BF16>::from_float(__builtin_fmaf((float)((w1 >> (8 * e)) & 0xffu), s, b));
  }
  return r;
}

// One chunk's registers as they arrive: K block bytes of tile j (tokens 16j +
// c), dims 64m + 16kg .. +15 (int8 and affine alike).
//   int8: V dims 16n + c at block positions 8kg .. +7 (n = 2h, 2h+1 in v[h]);
//     the K and V scales of positions 8kg .. 8kg+7.
//   affine: 4-bit V dims 16n + c at positions 8kg .. +7 (n = 4h .. 4h+3 in
//     v[h], dword n%4, nibble e = position 8kg + e); kx[2w + m] the K scale
//     (w 0) or bias (w 1) of group m for tokens c (low half) and 16 + c (high
//     half), whose slots s4_slot(block_pos(16j + c)) = 8(c/4) + 2(c%4) + j
//     make dword c of the group's row; vx[2w + g] the V scales (w 0) or biases
//     (w 1) of group g at slots 8kg .. 8kg+7 (positions (e, e+4) in dword e).
//   uint4: K bytes of token 16j + c, dims 64m + 16kg .. +15 for m = 0, 1 (one
//     16-byte run of the row, dword 2m + h = dims 64m + 16kg + 8h .. +7); V as
//     affine; kx[m] / kx[2 + m] the K scale / zero-point of group 2m + kg/2
//     for tokens c and 16 + c (dword c of the group's row); vx[g] / vz[g] the
//     V scales / zero-points of 32-dim group g at slots 8kg .. 8kg+7.
//   mixed pairs: the K part of one format with the V part of the other.
// Format pair FM = 4·KX + VX: K (KX) and V (VX) each 0 int8, 1 affine, 2 uint4.
constexpr int FX_I8 = 0, FX_AF = 1, FX_U4 = 2;
constexpr int FEW_I8 = 0, FEW_AF = 5, FEW_U4 = 10, FEW_I8U4 = 2, FEW_U4I8 = 8;
template <int KX>
struct FewK {  // int8: codes and the row scales
  v4i k[2][2];
  v4i ks;
};
template <>
struct FewK<FX_AF> {
  v4i k[2][2];
  v4i kx;
};
template <>
struct FewK<FX_U4> {
  v4i k4[2];
  v4i kx;
};
template <int VX>
struct FewV {  // int8: codes and the row scales
  v4i v[4];
  v4i vs;
};
template <>
struct FewV<FX_AF> {
  v4i v[2];
  v4i vx[4];
};
template <>
struct FewV<FX_U4> {
  v4i v[2];
  v4i vx[4], vz[4];
};
template <int FM>
struct FewChunk : FewK<FM / 4>, FewV<FM % 4> {};

template <int FM>
__device__ __forceinline__ void few_load(FewChunk<FM>& R, __amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv,
                                         __amdgpu_buffer_rsrc_t rks, __amdgpu_buffer_rsrc_t rvs,
                                         __amdgpu_buffer_rsrc_t rkz, __amdgpu_buffer_rsrc_t rvz,
                                         __amdgpu_buffer_rsrc_t none, bool ok, uint32_t blk, int c, int kg) {
  constexpr int KX = FM / 4, VX = FM % 4;
  const __amdgpu_buffer_rsrc_t a = ok ? rk : none, b = ok ? rv : none, sa = ok ? rks : none, sb = ok ? rvs : none;
  if constexpr (KX == FX_U4) {
    const __amdgpu_buffer_rsrc_t za = ok ? rkz : none;
#pragma unroll
    for (int j = 0; j < 2; ++j) R.k4[j] = ld128(a, (uint32_t)((16 * j + c) * 64 + 16 * kg), blk * 2048);
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const uint32_t off = (uint32_t)(64 * (2 * m + (kg >> 1)) + 4 * c);
      R.kx[m] = (int)ld32(sa, off, blk * 256);
      R.kx[2 + m] = (int)ld32(za, off, blk * 256);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int m = 0; m < 2; ++m) R.k[j][m] = ld128(a, (uint32_t)((16 * j + c) * 64 + 16 * kg + 2048 * m), blk * 4096);
    if constexpr (KX == FX_AF) {
#pragma unroll
      for (int w = 0; w < 4; ++w) R.kx[w] = (int)ld32(sa, (uint32_t)(64 * w + 4 * c), blk * 256);
    } else {
      R.ks = ld128(sa, (uint32_t)(16 * kg), blk * 64);
    }
  }
  if constexpr (VX == FX_I8) {
#pragma unroll
    for (int h = 0; h < 4; ++h) R.v[h] = ld128(b, (uint32_t)((c * 4 + kg) * 16 + 1024 * h), blk * 4096);
    R.vs = ld128(sb, (uint32_t)(16 * kg), blk * 64);
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) R.v[h] = ld128(b, (uint32_t)((c * 4 + kg) * 16 + 1024 * h), blk * 2048);
#pragma unroll
    for (int g = 0; g < 4; ++g) R.vx[g] = ld128(sb, (uint32_t)(64 * g + 16 * kg), blk * 256);
    if constexpr (VX == FX_U4) {
      const __amdgpu_buffer_rsrc_t zb = ok ? rvz : none;
#pragma unroll
      for (int g = 0; g < 4; ++g) R.vz[g] = ld128(zb, (uint32_t)(64 * g + 16 * kg), blk * 256);
    }
  }
}

template <bool BF16, int FM, int NT, bool EXACT, bool MH>  // MH: affine scales and biases in fp16
__global__ __launch_bounds__(64 * FW) void prefill_few_kernel(const PrefillArgs a) {
  constexpr int KX = FM / 4, VX = FM % 4;  // K and V formats
  typedef typename FewT<BF16>::vec V8;
  constexpr int NC = 16 * NT;  // (query, head) columns of the workgroup
  __shared__ __attribute__((aligned(16))) float part[FW][NC][FPR];
  __shared__ float pstat[FW][NC][2];
  const int tid = threadIdx.x, lane = tid & 63, c = lane & 15, kg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // workgroup 8 (n_rg u + r) + x is row group r of unit 8u + x, a unit being
  // a (split, KV head) pair (units past the last one: idle workgroups of
  // the grid's rounding)
  const int n_rg = (a.L * a.G + NC - 1) / NC;
  const int q8 = (int)blockIdx.x >> 3;
  const int rg = __builtin_amdgcn_readfirstlane(q8 % n_rg);
  const int unit = __builtin_amdgcn_readfirstlane(8 * (q8 / n_rg) + ((int)blockIdx.x & 7));
  if (unit >= a.S * a.Hkv) return;
  const int split = unit % a.S, h = unit / a.S, b = blockIdx.y;
  const int64_t bh = (int64_t)b * a.Hkv + h;
  const int p_base = rg * NC;                     // the group's first row
  const int rows = min(NC, a.L * a.G - p_base);  // and its row count (valid columns)
  const int P = (int)(a.T - a.L);
  const int64_t s_lo = a.split_lo + (int64_t)split * a.split_len;
  const int lo = __builtin_amdgcn_readfirstlane((int)s_lo);
  const int t_end = __builtin_amdgcn_readfirstlane((int)min(a.T, s_lo + a.split_len));

  // ---- the columns' query operands and causal limits ----
  V8 qop[NT][4];
  int qpos[NT];  // last visible token of the lane's column (causal), or past every token
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const bool valid = 16 * t + c < rows;
    const int p = p_base + 16 * t + c;
    const int qi = valid ? p / a.G : 0, hq = h * a.G + (valid ? p - qi * a.G : 0);
    qpos[t] = (valid && a.causal) ? P + qi : INT32_MAX;
    const uint16_t* row = (const uint16_t*)a.q + (int64_t)b * a.q_sb + (int64_t)hq * a.q_sh + (int64_t)qi * a.q_st;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int d0 = 64 * (ks >> 1) + 16 * kg + 8 * (ks & 1);
      v8s e = {0, 0, 0, 0, 0, 0, 0, 0};
      if (valid) {
        if (a.q_vec) {
          e = __builtin_bit_cast(v8s, *(const v4i*)(row + d0));
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) e[i] = (short)row[d0 + i];
        }
      }
      qop[t][ks] = __builtin_bit_cast(V8, e);
    }
  }

  // ---- resources of this (b, h) slice ----
  const int64_t cap = a.cap;
  constexpr int64_t KROW = KX == FX_U4 ? HEAD_DIM / 2 : HEAD_DIM;  // K code bytes per token
  constexpr int64_t VROW = VX == FX_I8 ? HEAD_DIM : HEAD_DIM / 2;  // V code bytes per token
  constexpr int64_t KSROW = KX == FX_I8 ? 1 : 4;                   // K scale entries per token
  constexpr int64_t VSROW = VX == FX_I8 ? 1 : 4;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc((const int8_t*)a.kq + bh * cap * KROW, cap * KROW);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc((const int8_t*)a.vq + bh * cap * VROW, cap * VROW);
  const __amdgpu_buffer_rsrc_t rks = make_rsrc(a.ks + bh * cap * KSROW, cap * KSROW * 2);
  const __amdgpu_buffer_rsrc_t rvs = make_rsrc(a.vs + bh * cap * VSROW, cap * VSROW * 2);
  const __amdgpu_buffer_rsrc_t none = make_rsrc(a.ks, 0);
  const __amdgpu_buffer_rsrc_t rkz = KX == FX_U4 ? make_rsrc(a.kz + bh * cap * 4, cap * 8) : none;
  const __amdgpu_buffer_rsrc_t rvz = VX == FX_U4 ? make_rsrc(a.vz + bh * cap * 4, cap * 8) : none;

  // ---- softmax state per column (log2 domain) ----
  // The running max starts at a finite floor, not -inf: a chunk whose tokens
  // all lie past a column's causal limit then gives p = exp2(-inf) = 0 for it
  // and no rescale, even as the wave's first chunk.
  constexpr float M_FLOOR = -1e30f;
  float m_run[NT], l_run[NT];
  v4f acc[NT][8];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    m_run[t] = M_FLOOR;
    l_run[t] = 0.f;
#pragma unroll
    for (int n = 0; n < 8; ++n) acc[t][n] = (v4f){0.f, 0.f, 0.f, 0.f};
  }

  const auto process = [&](const FewChunk<FM>& R, int t0) {
    // Q·Kᵀ: lane (c, kg) receives the scores of column c for tokens 16j + 4kg + i
    v4f s4[NT][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      V8 ka[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        if constexpr (KX == FX_U4) {
          // x̂ = (q - z)·s: the nibble unpack under the fp16 exponent of 1024
          // (64) and the zero-point plus that offset give q - z exactly in
          // fp16, bytes (0, 2) and (1, 3) of the dword as pairs; the product
          // with the fp16 scale is exact in fp32, rounded once to the query
          // dtype.  Elements in dim order: byte i holds dims 2i (low nibble), 2i+1.
          const int m = ks >> 1;
          const uint32_t w = (uint32_t)R.k4[j][ks], w8 = w >> 8;
          const uint32_t sw = (uint32_t)R.kx[m], zw = (uint32_t)R.kx[2 + m];
          const float sc = half_bits_to_float(j ? sw >> 16 : sw & 0xffffu);
          const _Float16 zh = __builtin_bit_cast(_Float16, (uint16_t)(j ? zw >> 16 : zw & 0xffffu));
          const v2h z1024 = {(_Float16)(zh + (_Float16)1024.0f), (_Float16)(zh + (_Float16)1024.0f)};
          const v2h z64 = {(_Float16)(zh + (_Float16)64.0f), (_Float16)(zh + (_Float16)64.0f)};
          const v2h lo02 = __builtin_bit_cast(v2h, and_or(w, 0x000f000fu, 0x64006400u)) - z1024;
          const v2h hi02 = __builtin_bit_cast(v2h, and_or(w, 0x00f000f0u, 0x54005400u)) - z64;
          const v2h lo13 = __builtin_bit_cast(v2h, and_or(w8, 0x000f000fu, 0x64006400u)) - z1024;
          const v2h hi13 = __builtin_bit_cast(v2h, and_or(w8, 0x00f000f0u, 0x54005400u)) - z64;
          const v2h pairs[4] = {lo02, hi02, lo13, hi13};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const v2h pr = pairs[e & 3];
            const _Float16 d = (e < 4) ? pr[0] : pr[1];  // bytes 0, 1 then 2, 3
            ka[ks][e] = FewT<BF16>::from_float(__builtin_fmaf((float)d, sc, 0.f));
          }
        } else {
          const v4i w = R.k[j][ks >> 1];
          if constexpr (KX == FX_AF) {
            const int m = ks >> 1;
            const uint32_t sw = (uint32_t)R.kx[m], bw = (uint32_t)R.kx[2 + m];
            const float sc = j ? meta_hi<MH>(sw) : meta_lo<MH>(sw);
            const float bi = j ? meta_hi<MH>(bw) : meta_lo<MH>(bw);
            ka[ks] = affine8<BF16>((uint32_t)w[2 * (ks & 1)], (uint32_t)w[2 * (ks & 1) + 1], sc, bi);
          } else {
            ka[ks] = FewT<BF16>::codes((uint32_t)w[2 * (ks & 1)], (uint32_t)w[2 * (ks & 1) + 1]);
          }
        }
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        v4f d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) d = FewT<BF16>::mfma(ka[ks], qop[t][ks], d);
        s4[t][j] = d;
      }
    }
    // the K row scale times the softmax scale, and the V scale, of the lane's
    // 8 positions (values formed in registers: the softmax scale alone, and P' = p)
    float ksm[8], vsf[8];
#pragma unroll
    for (int idx = 0; idx < 8; ++idx) {
      if constexpr (KX == FX_I8) ksm[idx] = half_at(R.ks, idx) * a.q_mul;
      else ksm[idx] = a.q_mul;
      if constexpr (VX == FX_I8) vsf[idx] = half_at(R.vs, idx);
      else vsf[idx] = 1.f;
    }
    // Range (as in the decode): a V scale of 2 or more among the lane's
    // positions makes its bound 0, so p <= 1 and P' = p·s stays finite in fp16
    bool big = false;
    if constexpr (VX == FX_I8) big = ((uint32_t)(R.vs[0] | R.vs[1] | R.vs[2] | R.vs[3]) & 0x40004000u) != 0;
    const float gap = big ? 0.f : RESCALE_GAP;
    // tokens past the split end or past a column's causal limit: only the
    // chunks at the end of the range (uniform test)
    const bool edge = t0 + FCH > t_end || t0 + FCH - 1 > P;
    // affine V under bf16 queries: V x̂ enters P·V as the bf16 value itself
    // (no widening to fp16) and P as bf16 high and low parts, positions
    // (e, e+4) at operand elements (2e, 2e+1), the order of the nibble unpack
    constexpr bool BPV = VX != FX_I8 && BF16;
    v8h pb[NT], pl[NT];  // pl: EXACT only
    v8bf ph[NT], plo[NT];  // BPV only
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      float x[8], pv[8];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) x[4 * j + i] = s4[t][j][i] * ksm[4 * j + i];
      if (edge) {
        const int last = min(qpos[t], t_end - 1) - t0 - 4 * kg;  // last visible token, relative
#pragma unroll
        for (int idx = 0; idx < 8; ++idx)
          if (16 * (idx >> 2) + (idx & 3) > last) x[idx] = NEG_INF;
      }
      float cmax = x[0];
#pragma unroll
      for (int idx = 1; idx < 8; ++idx) cmax = maxp(cmax, x[idx]);
      if (__ballot(cmax > m_run[t] + gap)) {
        cmax = max_xor32(max_xor16(cmax));  // the column's max over its four lanes
        const float m_new = fmaxf(m_run[t], cmax);
        const float f = __builtin_amdgcn_exp2f(m_run[t] - m_new);
        l_run[t] *= f;
#pragma unroll
        for (int n = 0; n < 8; ++n) acc[t][n] *= f;
        m_run[t] = m_new;
      }
#pragma unroll
      for (int idx = 0; idx < 8; idx += 2) {
        const float p0 = __builtin_amdgcn_exp2f(x[idx] - m_run[t]);
        const float p1 = __builtin_amdgcn_exp2f(x[idx + 1] - m_run[t]);
        l_run[t] += p0 + p1;
        if constexpr (BPV) {
          pv[idx] = p0;
          pv[idx + 1] = p1;
          continue;
        }
        // P' = p·s rounded to fp16 once (and, EXACT, its remainder)
        uint32_t w;
        asm("v_fma_mixlo_f16 %0, %1, %2, 0" : "=v"(w) : "v"(p0), "v"(vsf[idx]));
        asm("v_fma_mixhi_f16 %0, %1, %2, 0" : "+v"(w) : "v"(p1), "v"(vsf[idx + 1]));
        const v2h hh = __builtin_bit_cast(v2h, w);
        pb[t][idx] = hh[0];
        pb[t][idx + 1] = hh[1];
        if constexpr (EXACT) {
          pl[t][idx] = (_Float16)__builtin_fmaf(p0, vsf[idx], -(float)hh[0]);
          pl[t][idx + 1] = (_Float16)__builtin_fmaf(p1, vsf[idx + 1], -(float)hh[1]);
        }
      }
      if constexpr (BPV) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const v2bf hi = __builtin_convertvector((v2f){pv[e], pv[e + 4]}, v2bf);
          const v2bf lo = __builtin_convertvector((v2f){pv[e] - (float)hi[0], pv[e + 4] - (float)hi[1]}, v2bf);
          ph[t][2 * e] = hi[0];
          ph[t][2 * e + 1] = hi[1];
          plo[t][2 * e] = lo[0];
          plo[t][2 * e + 1] = lo[1];
        }
      }
    }
    // P·V
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      v8h va;
      v8bf vb;  // BPV
      if constexpr (VX == FX_U4) {
        // uint4 V: dims 16n + c sit in 32-dim group n / 2; (q - z)·s as in
        // the tiled kernel, positions (e, e+4) from dword e of the slot run
        const v2h k1024 = {(_Float16)1024.0f, (_Float16)1024.0f}, k64 = {(_Float16)64.0f, (_Float16)64.0f};
        const int g = n >> 1;
        const uint32_t W = (uint32_t)R.v[n >> 2][n & 3], W8 = W >> 8;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t sw = (uint32_t)R.vx[g][e], zw = (uint32_t)R.vz[g][e];
          const uint32_t t = (e & 1) ? and_or(e < 2 ? W : W8, 0x00f000f0u, 0x54005400u)
                                     : and_or(e < 2 ? W : W8, 0x000f000fu, 0x64006400u);
          const v2h d = __builtin_bit_cast(v2h, t) - (__builtin_bit_cast(v2h, zw) + ((e & 1) ? k64 : k1024));
          const v2h sv = __builtin_bit_cast(v2h, sw);
          const float x0 = __builtin_fmaf((float)d[0], (float)sv[0], 0.f);
          const float x1 = __builtin_fmaf((float)d[1], (float)sv[1], 0.f);
          if constexpr (BPV) {
            const v2bf xb = __builtin_convertvector((v2f){x0, x1}, v2bf);  // nearest even
            vb[2 * e] = xb[0];
            vb[2 * e + 1] = xb[1];
          } else {
            va[e] = FewT<BF16>::v_elem(x0);
            va[e + 4] = FewT<BF16>::v_elem(x1);
          }
        }
      } else if constexpr (VX == FX_AF) {
        // nibble e = position 8kg + e; the fp16 unpack under the exponent of
        // 1024 (64) yields the pair (e, e+4) exactly, whose scales and biases
        // share dword e of the slot run (s4_slot)
        const v2h k1024 = {(_Float16)1024.0f, (_Float16)1024.0f}, k64 = {(_Float16)64.0f, (_Float16)64.0f};
        const int g = n >> 2;
        const uint32_t W = (uint32_t)R.v[g][n & 3], W8 = W >> 8;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t sw = (uint32_t)R.vx[g][e], bw = (uint32_t)R.vx[2 + g][e];
          const uint32_t t = (e & 1) ? and_or(e < 2 ? W : W8, 0x00f000f0u, 0x54005400u)
                                     : and_or(e < 2 ? W : W8, 0x000f000fu, 0x64006400u);
          const v2h qv = __builtin_bit_cast(v2h, t) - ((e & 1) ? k64 : k1024);
          const float x0 = __builtin_fmaf((float)qv[0], meta_lo<MH>(sw), meta_lo<MH>(bw));
          const float x1 = __builtin_fmaf((float)qv[1], meta_hi<MH>(sw), meta_hi<MH>(bw));
          if constexpr (BPV) {
            const v2bf xb = __builtin_convertvector((v2f){x0, x1}, v2bf);  // nearest even
            vb[2 * e] = xb[0];
            vb[2 * e + 1] = xb[1];
          } else {
            va[e] = FewT<BF16>::v_elem(x0);
            va[e + 4] = FewT<BF16>::v_elem(x1);
          }
        }
      } else {
        va = i8x8_to_h8((uint32_t)R.v[n >> 1][2 * (n & 1)], (uint32_t)R.v[n >> 1][2 * (n & 1) + 1]);
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if constexpr (BPV) {
          acc[t][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vb, ph[t], acc[t][n], 0, 0, 0);
          acc[t][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vb, plo[t], acc[t][n], 0, 0, 0);
        } else {
          acc[t][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[t], acc[t][n], 0, 0, 0);
          if constexpr (EXACT) acc[t][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl[t], acc[t][n], 0, 0, 0);
        }
      }
    }
  };

  // ---- the wave's chunks w, w + 4, ... of [lo, t_end), a 2-deep ring ----
  const int n_chunks = (t_end - lo + FCH - 1) / FCH;
  const int n_w = n_chunks > wave ? (n_chunks - wave + FW - 1) / FW : 0;
  const uint32_t blk0 = (uint32_t)(lo / FCH + wave);
  FewChunk<FM> buf[2];
  few_load(buf[0], rk, rv, rks, rvs, rkz, rvz, none, 0 < n_w, blk0, c, kg);
  const int n_pad = (n_w + 1) / 2 * 2;
  for (int i0 = 0; i0 < n_pad; i0 += 2) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i = i0 + j;
      few_load(buf[(j + 1) & 1], rk, rv, rks, rvs, rkz, rvz, none, i + 1 < n_w, blk0 + FW * (i + 1), c, kg);
      if (i < n_w) process(buf[j], (int)(blk0 + FW * i) * FCH);
    }
  }

  // ---- wave partials -> LDS ----
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const float l = sum_xor32(sum_xor16(l_run[t]));
#pragma unroll
    for (int n = 0; n < 8; ++n) *(v4f*)&part[wave][16 * t + c][16 * n + 4 * kg] = acc[t][n];
    if (kg == 0) {
      pstat[wave][16 * t + c][0] = m_run[t];
      pstat[wave][16 * t + c][1] = l;
    }
  }
  __syncthreads();

  // ---- workgroup merge: thread (column, 4 dims) items ----
  for (int it = tid; it < rows * 32; it += 64 * FW) {
    const int p = it >> 5, d0 = 4 * (it & 31);
    float mw[FW], M = M_FLOOR;
#pragma unroll
    for (int w = 0; w < FW; ++w) {
      mw[w] = pstat[w][p][0];
      M = fmaxf(M, mw[w]);
    }
    v4f o = {0.f, 0.f, 0.f, 0.f};
    float l = 0.f;
#pragma unroll
    for (int w = 0; w < FW; ++w) {
      const float f = __builtin_amdgcn_exp2f(mw[w] - M);
      o += f * *(const v4f*)&part[w][p][d0];
      l += f * pstat[w][p][1];
    }
    const int pg = p_base + p;  // the row in the KV head's numbering
    const int qi = pg / a.G, hq = h * a.G + (pg - qi * a.G);
    if (a.S == 1) {
      if (a.sinks != nullptr) {
        const float sink = a.sinks[hq] * LOG2E;
        const float Mn = fmaxf(M, sink);
        const float f = __builtin_amdgcn_exp2f(M - Mn);
        l = l * f + __builtin_amdgcn_exp2f(sink - Mn);
        o *= f;
      }
      const v4f r = l > 0.f ? o * (1.f / l) : o;
      store_out4(a.out, (((int64_t)b * a.Hq + hq) * a.L + qi) * HEAD_DIM + d0, r, a.out_dtype);
    } else {
      // no visible key in this split: (-inf, 0, 0), as the tiled kernel writes
      const int64_t row = (((int64_t)bh * a.S + split) * a.nqb) * a.block_rows + pg;
      *(v4f*)(a.ws_acc + row * HEAD_DIM + d0) = o;
      if (d0 == 0) *(v2f*)(a.ws_stat + row * 2) = (v2f){l > 0.f ? M : NEG_INF, l};
    }
  }
}

template <bool BF16, int FM, bool EXACT, bool MH>
static void launch_nt(const PrefillArgs& a, int nt, dim3 grid, hipStream_t stream) {
  if (nt == 1) hipLaunchKernelGGL((prefill_few_kernel<BF16, FM, 1, EXACT, MH>), grid, dim3(64 * FW), 0, stream, a);
  else if (nt == 2) hipLaunchKernelGGL((prefill_few_kernel<BF16, FM, 2, EXACT, MH>), grid, dim3(64 * FW), 0, stream, a);
  else if (nt == 3) hipLaunchKernelGGL((prefill_few_kernel<BF16, FM, 3, EXACT, MH>), grid, dim3(64 * FW), 0, stream, a);
  else hipLaunchKernelGGL((prefill_few_kernel<BF16, FM, 4, EXACT, MH>), grid, dim3(64 * FW), 0, stream, a);
}

template <int FM, bool MH = false>
static void launch_fm(const PrefillArgs& a, int nt, bool exact, dim3 grid, hipStream_t stream) {
  if (a.q_dtype == DT_BF16) {
    if (exact) launch_nt<true, FM, true, MH>(a, nt, grid, stream);
    else launch_nt<true, FM, false, MH>(a, nt, grid, stream);
  } else {
    if (exact) launch_nt<false, FM, true, MH>(a, nt, grid, stream);
    else launch_nt<false, FM, false, MH>(a, nt, grid, stream);
  }
}

// Column tiles per workgroup: up to 32 of a launch's rows, row groups of one
// tile below 32,768 keys, else all the rows; 33-64 rows, groups of two tiles
// below 65,536 keys, else all the rows; above PREFILL_FEW_ROWS, groups of
// three tiles, or of four from 193 rows on.  32 q / 4 kv heads: two groups of
// one tile against one of two, 4 queries over 1K / 4K / 8K / 16K / 32K / 64K
// int8 keys 10.0 / 10.2 / 10.5 / 11.7 / 14.5 / 19.3 -> 8.1 / 8.3 / 8.9 / 10.5
// / 14.1 / 20.0 us, uint4 over 4K / 8K / 16K / 32K / 64K 11.5 / 12.1 / 13.2 /
// 16.6 / 22.6 -> 9.6 / 10.3 / 12.9 / 17.5 / 26.7 (affine alike); two groups
// of two tiles against one of four, 8 queries over 16K / 32K / 64K / 128K
// int8 keys 16.8 / 21.3 / 27.2 / 39.1 -> 13.3 / 18.3 / 25.8 / 40.7 us, uint4
// over 32K / 64K / 128K 24.1 / 33.4 / 50.5 -> 21.8 / 33.4 / 56.1, affine over
// 32K / 64K 23.7 / 32.3 -> 21.2 / 31.8 (6 queries over 64K: 26.4 -> 31.4).
int few_tiles(const PrefillArgs& a) {
  const int rows = a.L * a.G;
  if (rows <= 32) return rows > 16 && a.T < 32768 ? 1 : (rows + 15) / 16;
  if (rows <= PREFILL_FEW_ROWS) return a.T < 65536 ? 2 : (rows + 15) / 16;
  return rows <= 192 ? 3 : 4;
}

}  // namespace

// Up to PREFILL_FEW_ROWS rows the streaming kernel is the faster one at every
// cache length measured (33-64 rows below 65,536 keys in two row groups:
// 8 queries x 8 heads over 512 / 2K / 8K / 12K int8 keys, tiled -> streaming
// 14.2 / 14.3 / 14.6 / 14.3 -> 10.0 / 10.2 / 11.3 / 12.1 us; uint4 and affine
// over 4K 16.9 / 17.3 -> 11.7 / 11.4).  Row
// groups (more than 64 rows) from 16,384 to 131,071 keys; 32 q / 4 kv heads,
// tiled -> row groups: int8 12 queries over 32K 28.4 -> 22.0 us, 20 over 16K
// 26.6 -> 21.3, over 32K 36.4 -> 32.0, over 65,536 52.5 -> 49.4, 32 over 32K
// 41.8 -> 38.6 (20 over 131,072 keys 83.7 -> 86.7, hence the bound); uint4 K
// / int8 V 20 over 32K 36.4 -> 32.8, 12 over 65,536 43.5 -> 33.4.  A 4-bit V
// (uint4 or affine, its values formed in registers: the instruction-bound
// variants) gains only on small chunks and loses on larger ones (uint4 12
// over 32K 30.2 -> 27.5, 20 over 16K 28.6 -> 26.9, but 20 over 32K 37.4 ->
// 41.2 and over 65,536 57.3 -> 69.5; affine alike), hence its bound of
// 100 x 32,768 (row, key) pairs per KV head.
bool prefill_few_fits(const PrefillArgs& a) {
  const int rows = a.L * a.G;
  const bool fmt = ((a.k_fmt == 8 || a.k_fmt == 4) && (a.v_fmt == 8 || a.v_fmt == 4)) ||
                   (a.k_fmt == FMT_A8 && a.v_fmt == FMT_A4) || (a.k_fmt == FMT_A8H && a.v_fmt == FMT_A4H);
  const bool groups = rows <= PREFILL_BLOCK_ROWS && a.T >= 16384 && a.T < 131072 &&
                      (a.v_fmt == 8 || (int64_t)rows * a.T <= 100 * 32768);
  return fmt && a.window == 0 && a.bias.p == nullptr &&
         (rows <= PREFILL_FEW_ROWS || groups);
}

int prefill_few_groups(const PrefillArgs& a) {
  const int rows = a.L * a.G, nc = 16 * few_tiles(a);
  return (rows + nc - 1) / nc;
}

hipError_t launch_prefill_few(const PrefillArgs& a, hipStream_t stream) {
  const int nt = few_tiles(a);
  const int units = a.S * a.Hkv;
  const dim3 grid((unsigned)(8 * prefill_few_groups(a) * ((units + 7) / 8)), a.B);
  // the first query sees the fewest keys; from EXACT_PV_BELOW on, P' in one fp16 part
  const bool exact = (a.causal ? a.T - a.L + 1 : a.T) < EXACT_PV_BELOW;
  if (a.k_fmt == FMT_A8) launch_fm<FEW_AF>(a, nt, exact, grid, stream);
  else if (a.k_fmt == FMT_A8H) launch_fm<FEW_AF, true>(a, nt, exact, grid, stream);
  else if (a.k_fmt == 4 && a.v_fmt == 4) launch_fm<FEW_U4>(a, nt, exact, grid, stream);
  else if (a.k_fmt == 8 && a.v_fmt == 4) launch_fm<FEW_I8U4>(a, nt, exact, grid, stream);
  else if (a.k_fmt == 4 && a.v_fmt == 8) launch_fm<FEW_U4I8>(a, nt, exact, grid, stream);
  else launch_fm<FEW_I8>(a, nt, exact, grid, stream);
  return hipGetLastError();
}

}  // namespace rec
