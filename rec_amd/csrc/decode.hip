// Split-K flash decode over the quantized KV cache (gfx950).
//
// Restates, for this library's cache formats, the reference's decode path:
//   * quantized_attention_with_sinks (engine/src/rec_mlx/model.py:108-139):
//     scores = (q*scale)·k̂, per-head sink logit joins the softmax, out = P·v̂;
//   * the split-K partial (engine/src/rec_mlx/kernels/megakernel.py:619-693):
//     each split keeps a running max, a running sum and an fp32 accumulator;
//   * the merge (megakernel.py:276-318): top = max m_p, z = Σ e^{m_p-top} l_p,
//     out = Σ e^{m_p-top} acc_p / z (acc when z == 0);
//   * the append-then-attend order of Attention.__call__ (model.py:177-190),
//     fused here: the split that owns the newest token quantizes it first.
//
// Work decomposition.  Grid (splits, Hkv, B), 256 threads = 4 wavefronts.  A
// workgroup owns one KV head and a contiguous token range; its waves take
// 64-token chunks in turn.  All G <= 8 query heads of the KV head share every
// K/V byte loaded (GQA), so a K/V byte is read from HBM exactly once.
//
// Q·Kᵀ runs on v_mfma_i32_16x16x64_i8: the A operand is 16 cache rows of int8
// (int4: nibbles widened to bytes), the B operand is the query quantized to
// int16 and split into high and low int8 halves that fill the 16 columns
// (columns 0-7 = high halves of heads 0-7, 8-15 = low halves).  Integer
// products are exact; the two halves are recombined as 256*hi + lo with one
// DPP row rotation, then scaled by the row scale (and, for int4, corrected by
// the zero-point times the per-group query sum).  The int16 query keeps 15 bits
// of the query per head (relative error < 2^-16 of the head's largest
// element), well inside the 1e-3 output tolerance.
//
// P·V runs on v_mfma_f32_16x16x32_f16 with A = Vᵀ (16 dims × 32 tokens, exact
// small integers in fp16) and B = P'ᵀ where P' = p · v_scale is rounded to fp16
// once, as the reference rounds probabilities to the query dtype
// (model.py:132-133).  The token-blocked V layout makes each A operand one
// 16-byte load.  int4 V: P' carries each group's scale, the zero-point enters
// as a per-group correction Σ P'·z computed from the same rounded P'.
//
// Softmax runs in the log2 domain (log2(e) folded into the query scale).
#include "kernels.h"

namespace rec {


constexpr int MAX_SPLITS = DECODE_MAX_SPLITS;
constexpr int WAVES = 4;
constexpr float Q16 = 32512.0f;  // int16 query range: hi, lo stay inside int8

// LDS layout (bytes)
constexpr int LDS_QOP = 0;                         // up to 4 operands x 64 lanes x 16 B
constexpr int LDS_QSC = 4096;                      // 8 floats: per-head query scale
constexpr int LDS_QSUM = LDS_QSC + 32;             // 8 x 4 ints: per-group query sums (int4 K)
constexpr int LDS_FLAG = LDS_QSUM + 128;           // last-workgroup flag
constexpr int LDS_PART = 4352;                     // wave partials: 4 x 8 x 128 floats
constexpr int LDS_PSTAT = LDS_PART + WAVES * 8 * 128 * 4;  // 4 x 8 x (m, l)
constexpr int LDS_FSTAT = LDS_PART;                // final merge: S x 8 x (w, l), reuses partials
constexpr int LDS_BYTES = LDS_PSTAT + WAVES * 8 * 8;
static_assert(MAX_SPLITS * 8 * 8 <= WAVES * 8 * 128 * 4 + WAVES * 8 * 8, "final stats must fit");

// Order in which widen_u4() lays out 16 packed nibbles (8 bytes): unpacked byte
// j holds element perm16(j) of the 16.
__device__ __forceinline__ int u4_unpacked_pos(int o) { return (o & 8) + 4 * (o & 1) + ((o & 7) >> 1); }

__device__ __forceinline__ v4i widen_u4(v2i w) {
  const uint32_t w0 = (uint32_t)w[0], w1 = (uint32_t)w[1];
  v4i r;
  r[0] = (int)(w0 & 0x0f0f0f0fu);
  r[1] = (int)((w0 >> 4) & 0x0f0f0f0fu);
  r[2] = (int)(w1 & 0x0f0f0f0fu);
  r[3] = (int)((w1 >> 4) & 0x0f0f0f0fu);
  return r;
}

// Quantize this workgroup's G query rows to int16 (hi/lo int8) and lay them out
// as the B operands of the Q·Kᵀ MFMAs.
template <int KB>
__device__ void prepare_query(const DecodeArgs& a, int b, int h, char* smem, int tid) {
  int8_t* qop = (int8_t*)(smem + LDS_QOP);
  float* qsc = (float*)(smem + LDS_QSC);
  int* qsum = (int*)(smem + LDS_QSUM);
  if constexpr (KB == 4) {
    for (int i = tid; i < 1024; i += 256) ((int*)qop)[i] = 0;
    __syncthreads();
  }
  const int hh = tid >> 5, d0 = (tid & 31) * 4;
  float x[4] = {0.f, 0.f, 0.f, 0.f};
  if (hh < a.G) {
    const int64_t base = (int64_t)b * a.q_sb + (int64_t)(h * a.G + hh) * a.q_sh + d0;
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = load_as_float(a.q, base + i, a.q_dtype) * a.q_mul;
  }
  float amax = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
#pragma unroll
  for (int m = 1; m < 32; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
  const float inv = amax > 0.f ? Q16 / amax : 0.f;
  int gsum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int q16 = (int)__builtin_rintf(x[i] * inv);
    q16 = q16 > 32512 ? 32512 : (q16 < -32512 ? -32512 : q16);
    const int hi = (q16 + 128) >> 8;
    const int lo = q16 - hi * 256;
    gsum += q16;
    const int d = d0 + i;
    if constexpr (KB == 8) {
      const int m = d >> 6, kg = (d >> 4) & 3, j = d & 15;
      qop[(m * 64 + kg * 16 + hh) * 16 + j] = (int8_t)hi;
      qop[(m * 64 + kg * 16 + hh + 8) * 16 + j] = (int8_t)lo;
    } else {
      const int gg = d >> 5, pr = gg >> 1, o = d & 31;
      const int kg = 2 * (gg & 1) + (o >> 4), c = hh + 8 * (gg & 1), j = u4_unpacked_pos(o & 15);
      qop[((pr * 2 + 0) * 64 + kg * 16 + c) * 16 + j] = (int8_t)hi;
      qop[((pr * 2 + 1) * 64 + kg * 16 + c) * 16 + j] = (int8_t)lo;
    }
  }
  if constexpr (KB == 4) {
    // group of 32 dims = 8 consecutive threads
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) gsum += __shfl_xor(gsum, m, 64);
    if ((tid & 7) == 0) qsum[hh * 4 + ((tid & 31) >> 3)] = gsum;
  }
  if ((tid & 31) == 0) qsc[hh] = amax / Q16;
}

template <int KB, int VB>
__global__ __launch_bounds__(256) void decode_kernel(const DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[LDS_BYTES];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 15, kg = lane >> 4;
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int64_t bh = (int64_t)b * a.Hkv + h;
  const int64_t cap = a.cap;
  const int64_t t_begin = (int64_t)split * a.span;
  const int64_t t_end = t_begin + a.span < a.T ? t_begin + a.span : a.T;

  // Fused append of the newest token (position T-1) by the split that owns it.
  if (a.knew.p != nullptr && split == a.S - 1) {
    const int64_t pos = a.T - 1;
    if (wave == 0) {
      append_row<KB>(a.knew, b, h, 0, 0, (void*)a.kq, (uint16_t*)a.ks, (uint16_t*)a.kz, bh, cap, pos, lane);
    } else if (wave == 1) {
      if constexpr (VB == 8) {
        append_row<8>(a.vnew, b, h, 0, 1, (void*)a.vq, (uint16_t*)a.vs, nullptr, bh, cap, pos, lane);
      } else {
        const bool odd = (pos & 1) != 0;
        append_v4_pair(a.vnew, b, h, odd ? -1 : 0, !odd, odd, (uint8_t*)a.vq, (uint16_t*)a.vs, (uint16_t*)a.vz,
                       bh, cap, pos & ~(int64_t)1, lane);
      }
    }
    __threadfence_block();
  }

  prepare_query<KB>(a, b, h, smem, tid);
  __syncthreads();

  // Per-lane query operands and constants.
  constexpr int NOP = KB == 8 ? 2 : 4;
  v4i qop[NOP];
#pragma unroll
  for (int o = 0; o < NOP; ++o) qop[o] = ((const v4i*)(smem + LDS_QOP))[o * 64 + lane];
  const float qsc = ((const float*)(smem + LDS_QSC))[c & 7];
  int qsum_a = 0, qsum_b = 0;  // int4 K: per-group query sums of this lane's two groups
  if constexpr (KB == 4) {
    const int* qsum = (const int*)(smem + LDS_QSUM);
    qsum_a = qsum[(c & 7) * 4 + (c >> 3)];
    qsum_b = qsum[(c & 7) * 4 + 2 + (c >> 3)];
  }

  float m_run = NEG_INF, l_run = 0.f;
  v4f acc[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) acc[n] = (v4f){0.f, 0.f, 0.f, 0.f};
  float corr[4] = {0.f, 0.f, 0.f, 0.f};  // int4 V: Σ P'·z per group

  const int r = lane & 15;  // A-operand row of the Q·Kᵀ tiles
  for (int64_t t0 = t_begin + (int64_t)wave * BLOCK_T; t0 < t_end; t0 += WAVES * BLOCK_T) {
    // ---------------- loads ----------------
    // Q·Kᵀ tile j, row r holds token 16*(r>>2) + 4*j + (r&3) of the chunk, so
    // after four tiles lane (c, kg) holds the scores of tokens 16*kg .. 16*kg+15.
    v4i ka[4][2];
    if constexpr (KB == 8) {
      const int8_t* kbase = (const int8_t*)a.kq + (bh * cap + t0) * HEAD_DIM + 16 * kg;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tok = 16 * (r >> 2) + 4 * j + (r & 3);
        ka[j][0] = *(const v4i*)(kbase + tok * HEAD_DIM);
        ka[j][1] = *(const v4i*)(kbase + tok * HEAD_DIM + 64);
      }
    } else {
      const uint8_t* kbase = (const uint8_t*)a.kq + (bh * cap + t0) * (HEAD_DIM / 2) + 8 * kg;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tok = 16 * (r >> 2) + 4 * j + (r & 3);
        ka[j][0] = widen_u4(*(const v2i*)(kbase + tok * (HEAD_DIM / 2)));
        ka[j][1] = widen_u4(*(const v2i*)(kbase + tok * (HEAD_DIM / 2) + 32));
      }
    }
    // row scales of this lane's 16 tokens
    v4i ksr[2], kzr[2][2], ksr4[2][2];
    if constexpr (KB == 8) {
      const v4i* p = (const v4i*)(a.ks + bh * cap + t0 + 16 * kg);
      ksr[0] = p[0];
      ksr[1] = p[1];
    } else {
#pragma unroll
      for (int gi = 0; gi < 2; ++gi) {
        const int g = 2 * gi + (c >> 3);
        const int64_t off = bh * cap * 4 + (t0 >> 6) * (4 * BLOCK_T) + g * BLOCK_T + 16 * kg;
        ksr4[gi][0] = ((const v4i*)(a.ks + off))[0];
        ksr4[gi][1] = ((const v4i*)(a.ks + off))[1];
        kzr[gi][0] = ((const v4i*)(a.kz + off))[0];
        kzr[gi][1] = ((const v4i*)(a.kz + off))[1];
      }
    }
    // V: block n covers dims 16n..16n+15; lane (c, kg) gets dim 16n+c, tokens 16kg..16kg+15
    v4i va[8];
    v2i va4[8];
    if constexpr (VB == 8) {
      const int8_t* vbase = (const int8_t*)a.vq + bh * cap * HEAD_DIM + (t0 >> 6) * (BLOCK_T * HEAD_DIM) + c * BLOCK_T + 16 * kg;
#pragma unroll
      for (int n = 0; n < 8; ++n) va[n] = *(const v4i*)(vbase + n * 16 * BLOCK_T);
    } else {
      const uint8_t* vbase = (const uint8_t*)a.vq + bh * cap * (HEAD_DIM / 2) + (t0 >> 6) * (BLOCK_T * HEAD_DIM / 2) +
                             c * (BLOCK_T / 2) + 8 * kg;
#pragma unroll
      for (int n = 0; n < 8; ++n) va4[n] = *(const v2i*)(vbase + n * 16 * (BLOCK_T / 2));
    }
    v4i vsr[2], vsr4[4][2], vzr4[4][2];
    if constexpr (VB == 8) {
      const v4i* p = (const v4i*)(a.vs + bh * cap + t0 + 16 * kg);
      vsr[0] = p[0];
      vsr[1] = p[1];
    } else {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t off = bh * cap * 4 + (t0 >> 6) * (4 * BLOCK_T) + g * BLOCK_T + 16 * kg;
        vsr4[g][0] = ((const v4i*)(a.vs + off))[0];
        vsr4[g][1] = ((const v4i*)(a.vs + off))[1];
        vzr4[g][0] = ((const v4i*)(a.vz + off))[0];
        vzr4[g][1] = ((const v4i*)(a.vz + off))[1];
      }
    }

    // ---------------- scores ----------------
    float s[16];
    if constexpr (KB == 8) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v4i d = {0, 0, 0, 0};
        d = __builtin_amdgcn_mfma_i32_16x16x64_i8(ka[j][0], qop[0], d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_i32_16x16x64_i8(ka[j][1], qop[1], d, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int mine = d[i], partner = dpp_ror8(mine);
          const int full = c < 8 ? mine * 256 + partner : partner * 256 + mine;
          const int idx = 4 * j + i;
          const uint32_t sw = (uint32_t)ksr[idx >> 3][(idx & 7) >> 1];
          const float ksf = half_bits_to_float((idx & 1) ? (sw >> 16) : (sw & 0xffff));
          s[idx] = (float)full * (ksf * qsc);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v4i dah = {0, 0, 0, 0}, dal = {0, 0, 0, 0}, dbh = {0, 0, 0, 0}, dbl = {0, 0, 0, 0};
        dah = __builtin_amdgcn_mfma_i32_16x16x64_i8(ka[j][0], qop[0], dah, 0, 0, 0);
        dal = __builtin_amdgcn_mfma_i32_16x16x64_i8(ka[j][0], qop[1], dal, 0, 0, 0);
        dbh = __builtin_amdgcn_mfma_i32_16x16x64_i8(ka[j][1], qop[2], dbh, 0, 0, 0);
        dbl = __builtin_amdgcn_mfma_i32_16x16x64_i8(ka[j][1], qop[3], dbl, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int idx = 4 * j + i;
          const int sh = (idx & 1) ? 16 : 0;
          const float sa = half_bits_to_float(((uint32_t)ksr4[0][idx >> 3][(idx & 7) >> 1] >> sh) & 0xffff);
          const float za = half_bits_to_float(((uint32_t)kzr[0][idx >> 3][(idx & 7) >> 1] >> sh) & 0xffff);
          const float sb = half_bits_to_float(((uint32_t)ksr4[1][idx >> 3][(idx & 7) >> 1] >> sh) & 0xffff);
          const float zb = half_bits_to_float(((uint32_t)kzr[1][idx >> 3][(idx & 7) >> 1] >> sh) & 0xffff);
          const int ta = dah[i] * 256 + dal[i] - (int)za * qsum_a;
          const int tb = dbh[i] * 256 + dbl[i] - (int)zb * qsum_b;
          const float part = sa * (float)ta + sb * (float)tb;
          s[idx] = (part + dpp_ror8f(part)) * qsc;
        }
      }
    }
    // tokens past the split end
#pragma unroll
    for (int idx = 0; idx < 16; ++idx)
      if (t0 + 16 * kg + idx >= t_end) s[idx] = NEG_INF;

    // ---------------- online softmax ----------------
    float cmax = s[0];
#pragma unroll
    for (int idx = 1; idx < 16; ++idx) cmax = fmaxf(cmax, s[idx]);
    cmax = fmaxf(cmax, shfl_xor_f(cmax, 16));
    cmax = fmaxf(cmax, shfl_xor_f(cmax, 32));
    const float m_new = fmaxf(m_run, cmax);
    const float m_use = m_new == NEG_INF ? 0.f : m_new;
    const float factor = exp2f(m_run - m_use);
    float p[16], psum = 0.f;
#pragma unroll
    for (int idx = 0; idx < 16; ++idx) {
      p[idx] = exp2f(s[idx] - m_use);
      psum += p[idx];
    }
    l_run = l_run * factor + psum;
    m_run = m_new;
#pragma unroll
    for (int n = 0; n < 8; ++n) acc[n] *= factor;

    // ---------------- P·V ----------------
    if constexpr (VB == 8) {
      v8h pb[2];
#pragma unroll
      for (int idx = 0; idx < 16; ++idx) {
        const uint32_t sw = (uint32_t)vsr[idx >> 3][(idx & 7) >> 1];
        const float vsf = half_bits_to_float((idx & 1) ? (sw >> 16) : (sw & 0xffff));
        pb[idx >> 3][idx & 7] = (_Float16)(p[idx] * vsf);
      }
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        const v8h a0 = i8x8_to_h8((uint32_t)va[n][0], (uint32_t)va[n][1]);
        const v8h a1 = i8x8_to_h8((uint32_t)va[n][2], (uint32_t)va[n][3]);
        acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, pb[0], acc[n], 0, 0, 0);
        acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, pb[1], acc[n], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int g = 0; g < 4; ++g) corr[g] *= factor;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        v8h pb[2];
#pragma unroll
        for (int qq = 0; qq < 2; ++qq) {
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const int e = (k >> 1) + 4 * (k & 1);  // interleaved order of u4x8_to_h8_interleaved
            const int idx = 8 * qq + e;
            const int sh = (idx & 1) ? 16 : 0;
            const float vsf = half_bits_to_float(((uint32_t)vsr4[g][idx >> 3][(idx & 7) >> 1] >> sh) & 0xffff);
            const float vzf = half_bits_to_float(((uint32_t)vzr4[g][idx >> 3][(idx & 7) >> 1] >> sh) & 0xffff);
            const _Float16 ph = (_Float16)(p[idx] * vsf);
            pb[qq][k] = ph;
            corr[g] += (float)ph * vzf;
          }
        }
#pragma unroll
        for (int nn = 0; nn < 2; ++nn) {
          const int n = 2 * g + nn;
          const v8h a0 = u4x8_to_h8_interleaved((uint32_t)va4[n][0]);
          const v8h a1 = u4x8_to_h8_interleaved((uint32_t)va4[n][1]);
          acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, pb[0], acc[n], 0, 0, 0);
          acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, pb[1], acc[n], 0, 0, 0);
        }
      }
    }
  }

  // ---------------- wave partial -> LDS ----------------
  l_run += shfl_xor_f(l_run, 16);
  l_run += shfl_xor_f(l_run, 32);
  if constexpr (VB == 4) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      corr[g] += shfl_xor_f(corr[g], 16);
      corr[g] += shfl_xor_f(corr[g], 32);
    }
  }
  __syncthreads();  // query operands are no longer read; partial region is free
  float* part = (float*)(smem + LDS_PART);
  float* pstat = (float*)(smem + LDS_PSTAT);
  if (c < 8 && c < a.G) {
#pragma unroll
    for (int n = 0; n < 8; ++n)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = acc[n][i];
        if constexpr (VB == 4) v -= corr[n >> 1];
        part[(wave * 8 + c) * HEAD_DIM + 16 * n + 4 * kg + i] = v;
      }
    if (kg == 0) {
      pstat[(wave * 8 + c) * 2 + 0] = m_run;
      pstat[(wave * 8 + c) * 2 + 1] = l_run;
    }
  }
  __syncthreads();

  // ---------------- workgroup partial -> workspace ----------------
  const int hh = tid >> 5, d0 = (tid & 31) * 4;
  if (hh < a.G) {
    float mw[WAVES], M = NEG_INF;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      mw[w] = pstat[(w * 8 + hh) * 2];
      M = fmaxf(M, mw[w]);
    }
    v4f acc4 = {0.f, 0.f, 0.f, 0.f};
    float l = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const float f = mw[w] == NEG_INF ? 0.f : exp2f(mw[w] - M);
      acc4 += f * *(const v4f*)(part + (w * 8 + hh) * HEAD_DIM + d0);
      l += f * pstat[(w * 8 + hh) * 2 + 1];
    }
    const int64_t row = (bh * a.S + split) * 8 + hh;
    *(v4f*)(a.ws_acc + row * HEAD_DIM + d0) = acc4;
    if ((tid & 31) == 0) *(v2f*)(a.ws_stat + row * 2) = (v2f){M, l};
  }

  // ---------------- last workgroup of this KV head merges ----------------
  __threadfence();
  __syncthreads();
  int* flag = (int*)(smem + LDS_FLAG);
  if (tid == 0) flag[0] = atomicAdd(a.counters + bh, 1) == a.S - 1;
  __syncthreads();
  if (!flag[0]) return;
  __threadfence();

  float* fst = (float*)(smem + LDS_FSTAT);  // [S][8][2]: (m, l), then (weight, l)
  for (int i = tid; i < a.S * 8; i += 256) *(v2f*)(fst + 2 * i) = ((const v2f*)(a.ws_stat + bh * a.S * 16))[i];
  __syncthreads();
  const int sub = tid & 31;
  float lsum = 0.f;
  if (hh < a.G) {
    float M = NEG_INF;
    for (int sp = sub; sp < a.S; sp += 32) M = fmaxf(M, fst[(sp * 8 + hh) * 2]);
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) M = fmaxf(M, __shfl_xor(M, m, 64));
    float sink = NEG_INF;
    if (a.sinks != nullptr) {
      sink = a.sinks[h * a.G + hh] * LOG2E;
      M = fmaxf(M, sink);
    }
    for (int sp = sub; sp < a.S; sp += 32) {
      const float ms = fst[(sp * 8 + hh) * 2];
      const float w = (ms == NEG_INF || M == NEG_INF) ? 0.f : exp2f(ms - M);
      fst[(sp * 8 + hh) * 2] = w;
      lsum += w * fst[(sp * 8 + hh) * 2 + 1];
    }
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) lsum += __shfl_xor(lsum, m, 64);
    if (sink != NEG_INF) lsum += exp2f(sink - M);
  }
  __syncthreads();
  if (hh < a.G) {
    v4f acc4 = {0.f, 0.f, 0.f, 0.f};
    const float* src = a.ws_acc + (bh * a.S * 8 + hh) * HEAD_DIM + d0;
    int sp = 0;
    for (; sp + 8 <= a.S; sp += 8) {
      v4f v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = *(const v4f*)(src + (int64_t)(sp + u) * 8 * HEAD_DIM);
#pragma unroll
      for (int u = 0; u < 8; ++u) acc4 += fst[((sp + u) * 8 + hh) * 2] * v[u];
    }
    for (; sp < a.S; ++sp) acc4 += fst[(sp * 8 + hh) * 2] * *(const v4f*)(src + (int64_t)sp * 8 * HEAD_DIM);
    const v4f o = lsum > 0.f ? acc4 / lsum : acc4;
    *(v4f*)(a.out + ((int64_t)b * a.Hq + h * a.G + hh) * HEAD_DIM + d0) = o;
  }
  if (tid == 0) a.counters[bh] = 0;
}

hipError_t launch_decode(int kb, int vb, const DecodeArgs& a, hipStream_t stream) {
  const dim3 grid(a.S, a.Hkv, a.B), block(256);
  if (kb == 8 && vb == 8) hipLaunchKernelGGL((decode_kernel<8, 8>), grid, block, 0, stream, a);
  else if (kb == 8 && vb == 4) hipLaunchKernelGGL((decode_kernel<8, 4>), grid, block, 0, stream, a);
  else if (kb == 4 && vb == 8) hipLaunchKernelGGL((decode_kernel<4, 8>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((decode_kernel<4, 4>), grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace rec
