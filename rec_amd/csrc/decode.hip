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
// Each workgroup writes one partial (m, l, acc) per query head; a second
// kernel merges the splits, one workgroup per query head.
//
// Work decomposition.  Grid (splits, Hkv, B), 256 threads = 4 wavefronts.  A
// workgroup owns one KV head and a contiguous token range; its waves take
// 64-token chunks in turn, loading chunk i+1 while computing chunk i.  All G <= 8 query heads of the KV head share every
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
constexpr int LDS_QOP = 0;                                 // up to 4 operands x 64 lanes x 16 B
constexpr int LDS_QSC = 4096;                              // 8 floats: per-head query scale
constexpr int LDS_QSUM = LDS_QSC + 32;                     // 8 x 4 ints: per-group query sums (int4 K)
constexpr int LDS_PART = 4352;                             // wave partials: 4 x 8 x 128 floats
constexpr int LDS_PSTAT = LDS_PART + WAVES * 8 * 128 * 4;  // 4 x 8 x (m, l)
constexpr int LDS_BYTES = LDS_PSTAT + WAVES * 8 * 8;

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

// Tokens per compute chunk of one wave: one 32-token cache block.
constexpr int CH = BLOCK_T;

// Registers of one 32-token chunk as it arrives from HBM.  Members a format
// does not use are never touched and vanish.
struct Chunk {
  v4i k8[2][2];   // int8 K: tile j, MFMA half m (16 bytes each)
  v2i k4[2][2];   // int4 K: tile j, group pair (8 packed bytes each)
  v4i ks;         // int8 K: scales of this lane's 8 tokens
  v4i ks4[2];     // int4 K: scales, this lane's two groups
  v4i kz4[2];     // int4 K: zero-points
  v2i v8[8];      // int8 V: dim block n, this lane's 8 tokens
  uint32_t v4[8]; // int4 V: dim block n, this lane's 8 tokens packed
  v4i vs;         // int8 V: scales of this lane's 8 tokens
  v4i vs4[4];     // int4 V: scales, all four groups
  v4i vz4[4];     // int4 V: zero-points
};

struct Bases {
  const int8_t* k;     // this (b, h) slice of the K codes
  const int8_t* v;     // this (b, h) slice of the V codes
  const uint16_t* ks;  // K scales (int8: per token; int4: blocked per group)
  const uint16_t* kz;
  const uint16_t* vs;
  const uint16_t* vz;
};

__device__ __forceinline__ float half_at(const v4i& w, int idx) {
  const uint32_t x = (uint32_t)w[idx >> 1];
  return half_bits_to_float((idx & 1) ? (x >> 16) : (x & 0xffff));
}

template <class T>
__device__ __forceinline__ T ld_nt(const void* p) {
  return __builtin_nontemporal_load((const T*)p);
}

// Issue every load of the chunk (cache block) starting at token t0, a
// multiple of 32.  The KV cache is streamed once, so the loads are nontemporal.
template <int KB, int VB>
__device__ __forceinline__ void load_chunk(Chunk& R, const Bases& B, int t0, int lane) {
  const int c = lane & 15, kg = lane >> 4;
  const int blk = t0 >> 5;
  // Q·Kᵀ tile j, row r is token 16j + r of the block; the MFMA leaves lane
  // (c, kg) holding the scores of tokens 16j + 4kg + i, i.e. block positions
  // 8kg .. 8kg+7 in the order idx = 4j + i.
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    if constexpr (KB == 8) {
      const int8_t* p = B.k + blk * 4096 + (16 * j + c) * 64 + 16 * kg;
      R.k8[j][0] = ld_nt<v4i>(p);
      R.k8[j][1] = ld_nt<v4i>(p + 2048);
    } else {
      const int8_t* p = B.k + blk * 2048 + (16 * j + c) * 32 + 8 * kg;
      R.k4[j][0] = ld_nt<v2i>(p);
      R.k4[j][1] = ld_nt<v2i>(p + 1024);
    }
  }
  if constexpr (KB == 8) {
    R.ks = ld_nt<v4i>(B.ks + blk * 32 + 8 * kg);
  } else {
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      const int off = blk * 128 + (2 * gi + (c >> 3)) * 32 + 8 * kg;
      R.ks4[gi] = ld_nt<v4i>(B.ks + off);
      R.kz4[gi] = ld_nt<v4i>(B.kz + off);
    }
  }
  // V block n: lane (c, kg) gets dim 16n+c at block positions 8kg .. 8kg+7
  if constexpr (VB == 8) {
    const int8_t* p = B.v + blk * 4096 + c * 32 + 8 * kg;
#pragma unroll
    for (int n = 0; n < 8; ++n) R.v8[n] = ld_nt<v2i>(p + n * 512);
    R.vs = ld_nt<v4i>(B.vs + blk * 32 + 8 * kg);
  } else {
    const int8_t* p = B.v + blk * 2048 + c * 16 + 4 * kg;
#pragma unroll
    for (int n = 0; n < 8; ++n) R.v4[n] = ld_nt<uint32_t>(p + n * 256);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int off = blk * 128 + g * 32 + 8 * kg;
      R.vs4[g] = ld_nt<v4i>(B.vs + off);
      R.vz4[g] = ld_nt<v4i>(B.vz + off);
    }
  }
}

struct State {
  float m, l;     // running max (log2 domain) and sum of this lane's head
  v4f acc[8];     // P·V accumulators: dims 16n + 4kg + i of head c
  float corr[4];  // int4 V: Σ P'·z per group
};

template <int KB, int VB>
__device__ __forceinline__ void process_chunk(const Chunk& R, State& st, const v4i* qop, float qsc, int qsum_a,
                                              int qsum_b, int valid, int lane) {
  const int c = lane & 15, kg = lane >> 4;
  // ---------------- scores (log2 domain) ----------------
  float s[8];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    if constexpr (KB == 8) {
      v4i d = {0, 0, 0, 0};
      d = __builtin_amdgcn_mfma_i32_16x16x64_i8(R.k8[j][0], qop[0], d, 0, 0, 0);
      d = __builtin_amdgcn_mfma_i32_16x16x64_i8(R.k8[j][1], qop[1], d, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int mine = d[i], partner = dpp_ror8(mine);
        const int full = c < 8 ? mine * 256 + partner : partner * 256 + mine;
        s[4 * j + i] = (float)full * (half_at(R.ks, 4 * j + i) * qsc);
      }
    } else {
      const v4i ka = widen_u4(R.k4[j][0]), kb = widen_u4(R.k4[j][1]);
      v4i dah = {0, 0, 0, 0}, dal = {0, 0, 0, 0}, dbh = {0, 0, 0, 0}, dbl = {0, 0, 0, 0};
      dah = __builtin_amdgcn_mfma_i32_16x16x64_i8(ka, qop[0], dah, 0, 0, 0);
      dal = __builtin_amdgcn_mfma_i32_16x16x64_i8(ka, qop[1], dal, 0, 0, 0);
      dbh = __builtin_amdgcn_mfma_i32_16x16x64_i8(kb, qop[2], dbh, 0, 0, 0);
      dbl = __builtin_amdgcn_mfma_i32_16x16x64_i8(kb, qop[3], dbl, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int idx = 4 * j + i;
        const int ta = dah[i] * 256 + dal[i] - (int)half_at(R.kz4[0], idx) * qsum_a;
        const int tb = dbh[i] * 256 + dbl[i] - (int)half_at(R.kz4[1], idx) * qsum_b;
        const float part = half_at(R.ks4[0], idx) * (float)ta + half_at(R.ks4[1], idx) * (float)tb;
        s[idx] = (part + dpp_ror8f(part)) * qsc;
      }
    }
  }
  if (valid < CH) {  // tail chunk: tokens past the split end
#pragma unroll
    for (int idx = 0; idx < 8; ++idx)
      if (16 * (idx >> 2) + 4 * kg + (idx & 3) >= valid) s[idx] = NEG_INF;
  }

  // ---------------- online softmax ----------------
  float cmax = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
  cmax = fmaxf(cmax, shfl_xor_f(cmax, 16));
  cmax = fmaxf(cmax, shfl_xor_f(cmax, 32));
  const float m_new = fmaxf(st.m, cmax);
  if (__ballot(m_new > st.m)) {  // some head's max moved: rescale (rare after warm-up)
    const float factor = __builtin_amdgcn_exp2f(st.m - m_new);
    st.l *= factor;
#pragma unroll
    for (int n = 0; n < 8; ++n) st.acc[n] *= factor;
    if constexpr (VB == 4) {
#pragma unroll
      for (int g = 0; g < 4; ++g) st.corr[g] *= factor;
    }
    st.m = m_new;
  }
  float p[8];
#pragma unroll
  for (int idx = 0; idx < 8; ++idx) {
    p[idx] = __builtin_amdgcn_exp2f(s[idx] - st.m);
    st.l += p[idx];
  }

  // ---------------- P·V ----------------
  if constexpr (VB == 8) {
    v8h pb;
#pragma unroll
    for (int idx = 0; idx < 8; ++idx) pb[idx] = (_Float16)(p[idx] * half_at(R.vs, idx));
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      const v8h a0 = i8x8_to_h8((uint32_t)R.v8[n][0], (uint32_t)R.v8[n][1]);
      st.acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, pb, st.acc[n], 0, 0, 0);
    }
  } else {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      v8h pb;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int idx = (k >> 1) + 4 * (k & 1);  // order of u4x8_to_h8_interleaved
        const _Float16 ph = (_Float16)(p[idx] * half_at(R.vs4[g], idx));
        pb[k] = ph;
        st.corr[g] += (float)ph * half_at(R.vz4[g], idx);
      }
#pragma unroll
      for (int nn = 0; nn < 2; ++nn) {
        const int n = 2 * g + nn;
        st.acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(u4x8_to_h8_interleaved(R.v4[n]), pb, st.acc[n], 0, 0, 0);
      }
    }
  }
}

// Chunks in flight per wave: three for the int8 formats, two when int4
// scale/zero-point registers make a chunk larger.
template <int KB, int VB>
struct Depth {
  static constexpr int value = (KB == 8 && VB == 8) ? 3 : 2;
};

template <int KB, int VB>
__global__ __launch_bounds__(256) void decode_kernel(const DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[LDS_BYTES];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 15, kg = lane >> 4;
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int64_t bh = (int64_t)b * a.Hkv + h;
  const int64_t cap = a.cap;
  const bool fused = a.knew.p != nullptr;
  const bool tail = fused && split == a.S - 1;  // the split that owns the newest token
  int t_begin, t_end;
  if (tail) {
    t_begin = a.t_split_end;
    t_end = (int)a.T;
  } else {
    t_begin = split * a.span;
    t_end = t_begin + a.span < a.t_split_end ? t_begin + a.span : a.t_split_end;
  }

  Bases B;
  B.k = (const int8_t*)a.kq + bh * cap * (KB == 8 ? HEAD_DIM : HEAD_DIM / 2);
  B.v = (const int8_t*)a.vq + bh * cap * (VB == 8 ? HEAD_DIM : HEAD_DIM / 2);
  B.ks = a.ks + bh * cap * (KB == 8 ? 1 : 4);
  B.kz = KB == 4 ? a.kz + bh * cap * 4 : nullptr;
  B.vs = a.vs + bh * cap * (VB == 8 ? 1 : 4);
  B.vz = VB == 4 ? a.vz + bh * cap * 4 : nullptr;

  // Fused append of the newest token (position T-1), before this split reads it.
  if (tail) {
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
    __syncthreads();
  }

  // Start streaming before the query is prepared: the first chunks' loads
  // overlap the query load and quantization.
  constexpr int NBUF = Depth<KB, VB>::value;
  constexpr int STEP = WAVES * CH;
  Chunk buf[NBUF];
  int t = t_begin + wave * CH;
#pragma unroll
  for (int i = 0; i < NBUF - 1; ++i)
    if (t + i * STEP < t_end) load_chunk<KB, VB>(buf[i], B, t + i * STEP, lane);

  prepare_query<KB>(a, b, h, smem, tid);
  __syncthreads();

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

  State st;
  st.m = NEG_INF;
  st.l = 0.f;
#pragma unroll
  for (int n = 0; n < 8; ++n) st.acc[n] = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int g = 0; g < 4; ++g) st.corr[g] = 0.f;

  // Ring of NBUF chunk buffers, unrolled so every buffer index is static:
  // while buffer i is consumed, the loads of the chunk NBUF-1 ahead are in flight.
  bool more = t < t_end;
  while (more) {
#pragma unroll
    for (int i = 0; i < NBUF; ++i) {
      if (more) {
        const int ahead = t + (NBUF - 1) * STEP;
        if (ahead < t_end) load_chunk<KB, VB>(buf[(i + NBUF - 1) % NBUF], B, ahead, lane);
        process_chunk<KB, VB>(buf[i], st, qop, qsc, qsum_a, qsum_b, t_end - t, lane);
        t += STEP;
        more = t < t_end;
      }
    }
  }

  // ---------------- wave partial -> LDS ----------------
  st.l += shfl_xor_f(st.l, 16);
  st.l += shfl_xor_f(st.l, 32);
  if constexpr (VB == 4) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      st.corr[g] += shfl_xor_f(st.corr[g], 16);
      st.corr[g] += shfl_xor_f(st.corr[g], 32);
    }
  }
  float* part = (float*)(smem + LDS_PART);
  float* pstat = (float*)(smem + LDS_PSTAT);
  if (c < 8 && c < a.G) {
#pragma unroll
    for (int n = 0; n < 8; ++n)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = st.acc[n][i];
        if constexpr (VB == 4) v -= st.corr[n >> 1];
        part[(wave * 8 + c) * HEAD_DIM + 16 * n + 4 * kg + i] = v;
      }
    if (kg == 0) {
      pstat[(wave * 8 + c) * 2 + 0] = st.m;
      pstat[(wave * 8 + c) * 2 + 1] = st.l;
    }
  }
  __syncthreads();

  // ---------------- workgroup partial (or the output when S == 1) ----------------
  const int hh = tid >> 5, d0 = (tid & 31) * 4;
  if (hh < a.G) {
    float mw[WAVES], M = NEG_INF;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      mw[w] = pstat[(w * 8 + hh) * 2];
      M = fmaxf(M, mw[w]);
    }
    float sink = NEG_INF;
    if (a.S == 1 && a.sinks != nullptr) {
      sink = a.sinks[h * a.G + hh] * LOG2E;
      M = fmaxf(M, sink);
    }
    v4f acc4 = {0.f, 0.f, 0.f, 0.f};
    float l = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const float f = (mw[w] == NEG_INF || M == NEG_INF) ? 0.f : __builtin_amdgcn_exp2f(mw[w] - M);
      acc4 += f * *(const v4f*)(part + (w * 8 + hh) * HEAD_DIM + d0);
      l += f * pstat[(w * 8 + hh) * 2 + 1];
    }
    if (a.S == 1) {
      if (sink != NEG_INF) l += __builtin_amdgcn_exp2f(sink - M);
      const v4f o = l > 0.f ? acc4 / l : acc4;
      *(v4f*)(a.out + ((int64_t)b * a.Hq + h * a.G + hh) * HEAD_DIM + d0) = o;
    } else {
      const int64_t row = (bh * a.S + split) * 8 + hh;
      *(v4f*)(a.ws_acc + row * HEAD_DIM + d0) = acc4;
      if ((tid & 31) == 0) *(v2f*)(a.ws_stat + row * 2) = (v2f){M, l};
    }
  }
}

// Cross-split merge (megakernel.py:276-318): one workgroup per (query head,
// batch).  Thread (sg, d4) sums splits sg, sg+8, ... for dims 4*d4..4*d4+3;
// every partial load is issued before the first is used.
__global__ __launch_bounds__(256) void decode_merge_kernel(const DecodeArgs a) {
  __shared__ float red[8];
  __shared__ float wts[MAX_SPLITS];
  __shared__ v4f acc_part[8][32];
  const int tid = threadIdx.x, d4 = tid & 31, sg = tid >> 5;
  const int hq = blockIdx.x, b = blockIdx.y;
  const int h = hq / a.G, hh = hq % a.G;
  const int64_t bh = (int64_t)b * a.Hkv + h;
  const int S = a.S;
  constexpr int PER = MAX_SPLITS / 8;
  v4f v[PER];
  const float* src = a.ws_acc + ((bh * S) * 8 + hh) * HEAD_DIM + 4 * d4;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int sp = sg + 8 * i;
    v[i] = sp < S ? *(const v4f*)(src + (int64_t)sp * 8 * HEAD_DIM) : (v4f){0.f, 0.f, 0.f, 0.f};
  }
  float ms = NEG_INF, ls = 0.f;
  if (tid < S) {
    const v2f st = *(const v2f*)(a.ws_stat + ((bh * S + tid) * 8 + hh) * 2);
    ms = st[0];
    ls = st[1];
  }
  float M = wave_max(ms);
  if ((tid & 63) == 0) red[tid >> 6] = M;
  __syncthreads();
  M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float sink = NEG_INF;
  if (a.sinks != nullptr) {
    sink = a.sinks[hq] * LOG2E;
    M = fmaxf(M, sink);
  }
  const float w = (ms == NEG_INF || M == NEG_INF) ? 0.f : __builtin_amdgcn_exp2f(ms - M);
  if (tid < MAX_SPLITS) wts[tid] = w;
  float lw = w * ls;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) lw += __shfl_xor(lw, m, 64);
  __syncthreads();
  if ((tid & 63) == 0) red[4 + (tid >> 6)] = lw;
  v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int sp = sg + 8 * i;
    if (sp < S) acc += wts[sp] * v[i];
  }
  acc_part[sg][d4] = acc;
  __syncthreads();
  if (sg == 0) {
    float L = red[4] + red[5] + red[6] + red[7];
    if (sink != NEG_INF) L += __builtin_amdgcn_exp2f(sink - M);
    v4f t = acc_part[0][d4];
#pragma unroll
    for (int g = 1; g < 8; ++g) t += acc_part[g][d4];
    const v4f o = L > 0.f ? t / L : t;
    *(v4f*)(a.out + ((int64_t)b * a.Hq + hq) * HEAD_DIM + 4 * d4) = o;
  }
}

hipError_t launch_decode_partial(int kb, int vb, const DecodeArgs& a, hipStream_t stream) {
  const dim3 grid(a.S, a.Hkv, a.B), block(256);
  if (kb == 8 && vb == 8) hipLaunchKernelGGL((decode_kernel<8, 8>), grid, block, 0, stream, a);
  else if (kb == 8 && vb == 4) hipLaunchKernelGGL((decode_kernel<8, 4>), grid, block, 0, stream, a);
  else if (kb == 4 && vb == 8) hipLaunchKernelGGL((decode_kernel<4, 8>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((decode_kernel<4, 4>), grid, block, 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_decode_merge(const DecodeArgs& a, hipStream_t stream) {
  if (a.S == 1) return hipSuccess;  // the partial kernel wrote the output
  hipLaunchKernelGGL(decode_merge_kernel, dim3(a.Hq, a.B), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace rec
