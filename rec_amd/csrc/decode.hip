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
// Work decomposition.  Grid (splits, Hkv, B), 4 wavefronts (long uint4 splits: 8).  A
// workgroup owns one KV head and a contiguous token range; its waves take
// 32-token chunks in turn, loading chunk i+1 while computing chunk i.  All G <= 8 query heads of the KV head share every
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
// P·V runs on v_mfma_f32_16x16x32_f16: A = Vᵀ (16 dims × 32 tokens of exact
// small integers in fp16: int8 codes, 4-bit q - z, affine q) and B = P'ᵀ with
// P' = p · s the probability times the token's (group's) V scale, as an fp16
// high part in columns 0-7 and the rounding remainder in columns 8-15, which
// would otherwise repeat columns 0-7 (see EXACT_PV_BELOW for when the 4-bit
// and affine formats take the remainder).  The reference rounds probabilities
// to the query dtype before its P·V (model.py:132-133).  The token-blocked V
// layout makes each A operand one load per lane.
//
// Softmax runs in the log2 domain (log2(e) folded into the query scale).
#include "kernels.h"

namespace rec {


constexpr int MAX_SPLITS = DECODE_MAX_SPLITS;
constexpr float Q16 = 32512.0f;  // int16 query range: hi, lo stay inside int8

// Wavefronts per workgroup: four; uint4 K/V with long splits (>= 32 chunks,
// e.g. 131K tokens over 64 splits): eight, two per SIMD, because the nibble
// unpacking makes a 32-token chunk twice the VALU work per byte of int8 and a
// second wave per SIMD hides it (measured 3% faster at 131K tokens, slower
// at 32K and for the other formats).
constexpr int UINT4_WIDE_CHUNKS = 32;

// LDS layout (bytes) for W wavefronts
constexpr int LDS_QOP = 0;              // up to 4 operands x 64 lanes x 16 B
constexpr int LDS_QSC = 4096;           // 8 floats: per-head query scale
constexpr int LDS_QSUM = LDS_QSC + 32;  // 8 x 4 ints: per-group query sums (int4 K)
// A wave partial row holds 128 floats plus 4 of padding, so that the 8 query
// heads' rows start 4 banks apart and their stores do not collide on one bank.
constexpr int PART_ROW = HEAD_DIM + 4;
template <int W>
struct Lds {
  static constexpr int part = 4352;                  // wave partials: W x 8 rows of PART_ROW floats
  static constexpr int pstat = part + W * 8 * PART_ROW * 4;  // W x 8 x (m, l)
  static constexpr int meta = pstat + W * 8 * 8;        // int4: per wave [4 arrays][256 B] of one block
  static constexpr int bytes = meta + W * 1024;
};

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

// Raw bits of query elements i .. i+3 of a row whose dims are contiguous and
// whose start is 16-byte aligned (the host checks).  Two 8-byte loads, the
// second one only meaningful for fp32; no branch, so the compiler can leave the
// load in flight while the cache loads are issued behind it.
__device__ __forceinline__ v4i load_q_raw(const void* p, int64_t i, int dt) {
  const int es = dt == DT_F32 ? 4 : 2;
  const char* base = (const char*)p + i * es;
  const v2i w0 = *(const v2i*)base;
  const v2i w1 = *(const v2i*)(base + (es == 4 ? 8 : 0));
  return (v4i){w0[0], w0[1], w1[0], w1[1]};
}

__device__ __forceinline__ void q_raw_to_float(const v4i& r, int dt, float x[4]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t w = (uint32_t)r[k >> 1];
    const uint32_t bits = (k & 1) ? (w >> 16) : (w & 0xffffu);
    const float h16 = half_bits_to_float(bits), b16 = __builtin_bit_cast(float, bits << 16);
    const int rk = r[k];  // copy first: bit_cast of a vector subscript reads lane 0 in this clang
    const float f32 = __builtin_bit_cast(float, rk);
    x[k] = dt == DT_F32 ? f32 : (dt == DT_F16 ? h16 : b16);
  }
}

// Quantize this workgroup's G query rows to int16 (hi/lo int8) and lay them out
// as the B operands of the Q·Kᵀ MFMAs.  Thread (hh, d0) brings dims d0..d0+3 of
// head hh, already scaled (zero for hh >= G).
template <int KB, int NT>
__device__ void prepare_query(const float x[4], char* smem, int tid) {
  int8_t* qop = (int8_t*)(smem + LDS_QOP);
  float* qsc = (float*)(smem + LDS_QSC);
  int* qsum = (int*)(smem + LDS_QSUM);
  if constexpr (KB == 4) {
    for (int i = tid; i < 1024; i += NT) ((int*)qop)[i] = 0;
    __syncthreads();
  }
  if (tid >= 256) return;  // threads (hh, d0) cover 8 heads x 128 dims
  const int hh = tid >> 5, d0 = (tid & 31) * 4;
  float amax = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
  amax = max_xor16(row16_max(amax));  // the 32 lanes of head hh
  const float inv = amax > 0.f ? Q16 / amax : 0.f;
  int gsum = 0;
  uint32_t hi4 = 0, lo4 = 0;  // int8 K: the four dims' bytes, stored as one dword each
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int q16 = (int)__builtin_rintf(x[i] * inv);
    q16 = q16 > 32512 ? 32512 : (q16 < -32512 ? -32512 : q16);
    const int hi = (q16 + 128) >> 8;
    const int lo = q16 - hi * 256;
    gsum += q16;
    const int d = d0 + i;
    if constexpr (KB == 8 || is_a8(KB)) {
      hi4 |= (uint32_t)(hi & 0xff) << (8 * i);
      lo4 |= (uint32_t)(lo & 0xff) << (8 * i);
    } else {
      const int gg = d >> 5, pr = gg >> 1, o = d & 31;
      const int kg = 2 * (gg & 1) + (o >> 4), c = hh + 8 * (gg & 1), j = u4_unpacked_pos(o & 15);
      qop[((pr * 2 + 0) * 64 + kg * 16 + c) * 16 + j] = (int8_t)hi;
      qop[((pr * 2 + 1) * 64 + kg * 16 + c) * 16 + j] = (int8_t)lo;
    }
  }
  if constexpr (KB == 8 || is_a8(KB)) {
    // dims d0 .. d0+3 share operand m and lane row kg*16 + hh; bytes j .. j+3
    const int m = d0 >> 6, kg = (d0 >> 4) & 3, j = d0 & 15;
    *(uint32_t*)(qop + (m * 64 + kg * 16 + hh) * 16 + j) = hi4;
    *(uint32_t*)(qop + (m * 64 + kg * 16 + hh + 8) * 16 + j) = lo4;
  }
  if constexpr (KB == 4 || is_a8(KB)) {
    // group of 32 dims = 8 consecutive threads
    gsum = group8_sum(gsum);
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
  v4i k4[2];      // int4 K: tile j, both halves (8 packed bytes each)
  v4i v8[4];      // int8 V: dim blocks 2h, 2h+1 (8 bytes each), this lane's 8 tokens
  v4i v4[2];      // int4 V: dim blocks 4h..4h+3, this lane's 8 tokens packed
  v4i s8[2];      // int8 scales of this lane's 8 positions: [0] K, [1] V
  v4i m4;         // uint4 K and V: the block's four metadata arrays (K scales, K
                  // zeros, V scales, V zeros), 16 bytes per lane: lanes 16a .. 16a+15
                  // hold array a; handed out through LDS
  uint32_t m[4];  // one 4-bit side's (or the affine format's) metadata, one dword per
                  // lane: [0] K scales, [1] K zeros, [2] V scales, [3] V zeros;
                  // handed out through LDS
};

// Buffer resources of one (b, h) slice of the cache, plus an empty one.  Every
// chunk load goes through them: a chunk slot a wave does not own loads through
// the empty resource (zeros, no memory access) but is issued all the same, which
// keeps every load unconditional and lets the compiler count the loads in
// flight exactly (a load under a branch makes it drain them all).  Block
// offsets travel in the scalar soffset operand and the per-lane offsets are
// loop-invariant registers.  Range checks need not cover soffset: the empty
// resource has no records, so any lane offset is out of range and reads zero,
// and real loads stay inside their slice.
struct Res {
  __amdgpu_buffer_rsrc_t k, v, ks, kz, vs, vz, none;
};

// Per-lane byte offsets inside a cache block (fixed for the whole kernel).
struct LaneOff {
  uint32_t k[2];  // K codes, tile j (int8: the second MFMA half is +2048)
  uint32_t v;     // V codes, run h at +1024 h
  uint32_t s8;    // int8 scales of this lane's positions 8kg .. 8kg+7
  uint32_t m4;    // int4 scale / zero-point dword of this lane
};

template <int KB, int VB>
__device__ __forceinline__ LaneOff lane_offsets(int lane) {
  const int c = lane & 15, kg = lane >> 4;
  LaneOff o;
#pragma unroll
  for (int j = 0; j < 2; ++j) o.k[j] = (16 * j + c) * 64 + 16 * kg;
  o.v = (c * 4 + kg) * 16;
  o.s8 = 16 * kg;
  o.m4 = 4 * lane;
  return o;
}

// Issue every load of cache block `blk` of the slice, or (ok false) the same
// loads through the empty resource.  uint4 K and V bring the block's metadata
// in one 16-byte load per lane from `mbase` (the lane's own array and
// offset; block 0 when ok is false), instead of four 4-byte loads: 3% faster
// at 32K and 131K tokens.
template <int KB, int VB>
__device__ __forceinline__ void load_chunk(Chunk& R, const Res& S, const LaneOff& o, bool ok, uint32_t blk,
                                           const char* mbase) {
  const __amdgpu_buffer_rsrc_t rk = ok ? S.k : S.none, rks = ok ? S.ks : S.none, rkz = ok ? S.kz : S.none;
  const __amdgpu_buffer_rsrc_t rv = ok ? S.v : S.none, rvs = ok ? S.vs : S.none, rvz = ok ? S.vz : S.none;
  // Q·Kᵀ tile j, row r is token 16j + r of the block; the MFMA leaves lane
  // (c, kg) holding the scores of tokens 16j + 4kg + i, i.e. block positions
  // 8kg .. 8kg+7 in the order idx = 4j + i.
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    if constexpr (KB == 8 || is_a8(KB)) {
      R.k8[j][0] = ld128(rk, o.k[j], blk * 4096);
      R.k8[j][1] = ld128(rk, o.k[j] + 2048, blk * 4096);
    } else {
      R.k4[j] = ld128(rk, o.k[j], blk * 2048);
    }
  }
  if constexpr (KB == 4 && VB == 4) {
    R.m4 = __builtin_nontemporal_load((const v4i*)(mbase + (size_t)(ok ? blk : 0u) * 256));
  } else if constexpr (KB == 8) {
    R.s8[0] = ld128(rks, o.s8, blk * 64);
  } else if constexpr (is_a8(KB)) {
    R.m[0] = ld32(rks, o.m4, blk * 256);  // scales and biases
  } else {
    R.m[0] = ld32(rks, o.m4, blk * 256);
    R.m[1] = ld32(rkz, o.m4, blk * 256);
  }
  // V: lane (c, kg) gets dims 16n+c at block positions 8kg .. 8kg+7
  if constexpr (VB == 8) {
#pragma unroll
    for (int h = 0; h < 4; ++h) R.v8[h] = ld128(rv, o.v + h * 1024, blk * 4096);
    R.s8[1] = ld128(rvs, o.s8, blk * 64);
  } else {
    R.v4[0] = ld128(rv, o.v, blk * 2048);
    R.v4[1] = ld128(rv, o.v + 1024, blk * 2048);
    if constexpr (KB != 4 || VB != 4) {
      R.m[2] = ld32(rvs, o.m4, blk * 256);  // affine: scales and biases
      if constexpr (VB == 4) R.m[3] = ld32(rvz, o.m4, blk * 256);
    }
  }
}

struct State {
  float m, l;     // running max (log2 domain) and sum of this lane's head
  v4f acc[8];     // P·V accumulators: dims 16n + 4kg + i of head c
  float vb[2];    // affine V: Σ p·bias over this lane's tokens, per 64-dim group
};

// bf16 (F16: fp16) element `slot` of 8 packed in a v4i, as float
template <bool F16>
__device__ __forceinline__ float meta_at(const v4i& w, int slot) {
  const uint32_t x = (uint32_t)w[slot >> 1];
  return (slot & 1) ? meta_hi<F16>(x) : meta_lo<F16>(x);
}

template <int KB, int VB, bool EXACT, bool MASK>
__device__ __forceinline__ void process_chunk(const Chunk& R, State& st, const v4i* qop, float qsc, float qsum_a,
                                              float qsum_b, int valid, int lane, char* meta, const v4i* bz,
                                              float bmul) {
  const int c = lane & 15, kg = lane >> 4;
  // int8 scales arrive as the lane's own 16-byte run (positions 8kg ..
  // 8kg+7).  int4 scales and zero-points arrive one dword per lane; this
  // wavefront's LDS region ([K scales][K zeros][V scales][V zeros], 256 B
  // each, [4 groups][32 slots]) hands each lane the 16-byte runs it needs.
  // Affine formats use the K and V halves of the region as [scales g0 g1][biases g0 g1].
  v4i ks, vs, ks4[2], kz4[2], vs4[4], vz4[4];
  if constexpr (KB == 8) ks = R.s8[0];
  if constexpr (VB == 8) vs = R.s8[1];
  if constexpr (KB == 4 || VB == 4 || is_a8(KB) || is_a4(VB)) {
    uint32_t* mw = (uint32_t*)meta;
    if constexpr (KB == 4 && VB == 4) {
      // lanes 48-63 carry the V zero-points, dword e of a run being the pair
      // of unpack step e: the unpack's exponent offsets (1024 for even e, 64
      // for odd) are added here once instead of per group in every lane
      v4i m4 = R.m4;
      const bool vz_lane = lane >= 48;
      const v2h o_even = vz_lane ? (v2h){(_Float16)1024.0f, (_Float16)1024.0f} : (v2h){(_Float16)0.0f, (_Float16)0.0f};
      const v2h o_odd = vz_lane ? (v2h){(_Float16)64.0f, (_Float16)64.0f} : (v2h){(_Float16)0.0f, (_Float16)0.0f};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int x = m4[e];  // a copy: a bit_cast of a vector subscript reads element 0
        m4[e] = __builtin_bit_cast(int, __builtin_bit_cast(v2h, x) + ((e & 1) ? o_odd : o_even));
      }
      *(v4i*)(meta + 16 * lane) = m4;  // array lane / 16, bytes 16 (lane % 16) ..
    } else if constexpr (KB == 4) {
      mw[lane] = R.m[0];
      mw[64 + lane] = R.m[1];
    }
    if constexpr (is_a8(KB)) mw[lane] = R.m[0];
    if constexpr (VB == 4 && KB != 4) {
      mw[128 + lane] = R.m[2];
      // the V zero-points with the unpack's exponent offset of their step e = lane % 4
      const v2h off = (lane & 1) ? (v2h){(_Float16)64.0f, (_Float16)64.0f} : (v2h){(_Float16)1024.0f, (_Float16)1024.0f};
      mw[192 + lane] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2h, R.m[3]) + off);
    }
    if constexpr (is_a4(VB)) mw[128 + lane] = R.m[2];
    wave_lds_sync();
    if constexpr (is_a8(KB)) {
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        ks4[g] = *(const v4i*)(meta + g * 64 + 16 * kg);        // scales, slots 8kg .. 8kg+7
        kz4[g] = *(const v4i*)(meta + 128 + g * 64 + 16 * kg);  // biases
      }
    }
    if constexpr (is_a4(VB)) {
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        vs4[g] = *(const v4i*)(meta + 512 + g * 64 + 16 * kg);
        vz4[g] = *(const v4i*)(meta + 640 + g * 64 + 16 * kg);
      }
    }
    if constexpr (KB == 4) {
#pragma unroll
      for (int gi = 0; gi < 2; ++gi) {
        const int off = (2 * gi + (c >> 3)) * 64 + 16 * kg;  // this lane's groups: 2gi + (c >= 8)
        ks4[gi] = *(const v4i*)(meta + off);
        kz4[gi] = *(const v4i*)(meta + 256 + off);
      }
    }
    if constexpr (VB == 4) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        vs4[g] = *(const v4i*)(meta + 512 + g * 64 + 16 * kg);
        vz4[g] = *(const v4i*)(meta + 768 + g * 64 + 16 * kg);
      }
    }
  }
  // ---------------- scores ----------------
  // In units of the query quantization step: the step (qsc) is applied in the
  // exponent below, where it costs an fma instead of a multiply per score.
  float s[8];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    if constexpr (KB == 8) {
      v4i d = {0, 0, 0, 0};
      d = __builtin_amdgcn_mfma_i32_16x16x64_i8(R.k8[j][0], qop[0], d, 0, 0, 0);
      d = __builtin_amdgcn_mfma_i32_16x16x64_i8(R.k8[j][1], qop[1], d, 0, 0, 0);
      // columns c < 8 hold the high query byte, c + 8 the low one: the lane
      // weights its own sum and its partner's by 256 and 1 (or 1 and 256)
      const int sh_mine = c < 8 ? 8 : 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int mine = d[i], partner = dpp_ror8(mine);
        const int full = (mine << sh_mine) + (partner << (8 - sh_mine));
        s[4 * j + i] = (float)full * half_at(ks, 4 * j + i);
      }
    } else if constexpr (is_a8(KB)) {
      // uint8 codes k enter as k - 128 (top bit flipped), one MFMA per 64-dim
      // group: Σ q (s k + b) = s·Σ q (k - 128) + (128 s + b)·Q over the group,
      // Q = the group's query sum (exact)
      const v4i flip = {(int)0x80808080u, (int)0x80808080u, (int)0x80808080u, (int)0x80808080u};
      v4i d0 = {0, 0, 0, 0}, d1 = {0, 0, 0, 0};
      d0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(R.k8[j][0] ^ flip, qop[0], d0, 0, 0, 0);
      d1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(R.k8[j][1] ^ flip, qop[1], d1, 0, 0, 0);
      const int sh_mine = c < 8 ? 8 : 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int sl = 2 * i + j;  // slot of position 4j + i
        const int m0 = d0[i], p0 = dpp_ror8(m0), m1 = d1[i], p1 = dpp_ror8(m1);
        const float f0 = (float)((m0 << sh_mine) + (p0 << (8 - sh_mine)));
        const float f1 = (float)((m1 << sh_mine) + (p1 << (8 - sh_mine)));
        constexpr bool F16 = meta_f16(KB);
        const float s0 = meta_at<F16>(ks4[0], sl), s1 = meta_at<F16>(ks4[1], sl);
        const float c0 = fmaf(128.f, s0, meta_at<F16>(kz4[0], sl)), c1 = fmaf(128.f, s1, meta_at<F16>(kz4[1], sl));
        s[4 * j + i] = fmaf(s0, f0, fmaf(s1, f1, fmaf(c0, qsum_a, c1 * qsum_b)));
      }
    } else {
      const v4i ka = widen_u4((v2i){R.k4[j][0], R.k4[j][1]}), kb = widen_u4((v2i){R.k4[j][2], R.k4[j][3]});
      v4i dah = {0, 0, 0, 0}, dal = {0, 0, 0, 0}, dbh = {0, 0, 0, 0}, dbl = {0, 0, 0, 0};
      dah = __builtin_amdgcn_mfma_i32_16x16x64_i8(ka, qop[0], dah, 0, 0, 0);
      dal = __builtin_amdgcn_mfma_i32_16x16x64_i8(ka, qop[1], dal, 0, 0, 0);
      dbh = __builtin_amdgcn_mfma_i32_16x16x64_i8(kb, qop[2], dbh, 0, 0, 0);
      dbl = __builtin_amdgcn_mfma_i32_16x16x64_i8(kb, qop[3], dbl, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int idx = 4 * j + i, sl = 2 * i + j;  // position idx of the lane's run sits at slot sl
        // Σ (k - z) q over one 32-dim group: the high/low byte sums combine
        // exactly in int32; |k - z| <= 15 and |q| <= 32512 keep every float
        // intermediate an integer below 2^24, so the fma is exact too
        const float ta = fmaf(-half_at(kz4[0], sl), qsum_a, (float)((dah[i] << 8) + dal[i]));
        const float tb = fmaf(-half_at(kz4[1], sl), qsum_b, (float)((dbh[i] << 8) + dbl[i]));
        const float part = fmaf(half_at(ks4[0], sl), ta, half_at(ks4[1], sl) * tb);
        s[idx] = part + dpp_ror8f(part);
      }
    }
  }
  // MASK: the bias of the lane's tokens 16j + 4kg + i (bz[j][i], natural
  // log units) joins each score, in the score's units (bmul = log2 e / qsc);
  // -inf drops the token
  if constexpr (MASK) {
#pragma unroll
    for (int idx = 0; idx < 8; ++idx) {
      const int w = bz[idx >> 2][idx & 3];  // a copy: a bit_cast of a vector subscript reads element 0
      s[idx] = __builtin_fmaf(__builtin_bit_cast(float, w), bmul, s[idx]);
    }
  }
  // tail chunk: tokens past the split end (rare: without the hint the
  // compiler turns this into compares and selects on every chunk)
  if (__builtin_expect(valid < CH, 0)) {
#pragma unroll
    for (int idx = 0; idx < 8; ++idx)
      if (16 * (idx >> 2) + 4 * kg + (idx & 3) >= valid) s[idx] = NEG_INF;
  }

  // ---------------- online softmax (log2 domain: score * qsc) ----------------
  // The running max moves only when a score exceeds it by more than
  // RESCALE_GAP: probabilities up to 2^RESCALE_GAP are as exact in the fp16
  // operands and fp32 sums as ones up to 1.  A head's max over the chunk
  // exceeds the bound iff one of its four lanes' own maxima does, so the
  // cross-lane reduction and the rescale run only then (after the first
  // chunk, rarely).
  //
  // Range: the fp16 operand p·s stays finite while p·|s| < 65504.  A V scale
  // of 2 or more (fp16 / bf16 exponent bit 14; int8 |v| >= 254, a 4-bit
  // group range >= 30) makes the chunk's gap 0 for the lanes that hold it
  // (int8: the lane's own eight scales; 4-bit and affine: any scale of the
  // block, a wave vote), so their p <= 1 and p·|s| <= |s| <= 65504 (fp16
  // scales; an affine bf16 scale above that is out of range).
  bool big;
  if constexpr (VB == 8) {
    big = ((uint32_t)(vs[0] | vs[1] | vs[2] | vs[3]) & 0x40004000u) != 0;
  } else if constexpr (is_a4(VB)) {
    big = __ballot(lane < 32 && (R.m[2] & 0x40004000u) != 0) != 0;  // lanes 32-63 hold biases
  } else if constexpr (KB == 4) {
    const uint32_t w = (uint32_t)(R.m4[0] | R.m4[1] | R.m4[2] | R.m4[3]);
    big = __ballot((lane >> 4) == 2 && (w & 0x40004000u) != 0) != 0;  // lanes 32-47 hold the V scales
  } else {
    big = __ballot((R.m[2] & 0x40004000u) != 0) != 0;
  }
  const float gap = big ? 0.f : RESCALE_GAP;
  float cmax = s[0];
#pragma unroll
  for (int idx = 1; idx < 8; ++idx) cmax = maxp(cmax, s[idx]);
  cmax *= qsc;  // qsc > 0
  if (__ballot(cmax > st.m + gap)) {
    cmax = max_xor32(max_xor16(cmax));
    const float m_new = fmaxf(st.m, cmax);
    // 0 on the first chunk, 1 if unchanged (MASK: a head whose every score so
    // far is -inf keeps m = -inf and zero sums)
    const float factor = MASK && st.m == NEG_INF ? 0.f : __builtin_amdgcn_exp2f(st.m - m_new);
    st.l *= factor;
    if constexpr (is_a4(VB)) {
      st.vb[0] *= factor;
      st.vb[1] *= factor;
    }
#pragma unroll
    for (int n = 0; n < 8; ++n) st.acc[n] *= factor;
    st.m = m_new;
  }
  float p[8];
  // MASK: while a head's running max is still -inf every score it has seen is
  // -inf, and p = exp2(-inf - 0) = 0 (not exp2(NaN))
  const float moff = MASK && st.m == NEG_INF ? 0.f : st.m;
#pragma unroll
  for (int idx = 0; idx < 8; ++idx) {
    p[idx] = __builtin_amdgcn_exp2f(fmaf(s[idx], qsc, -moff));
    st.l += p[idx];
  }

  // ---------------- P·V ----------------
  // The B operand carries P' = p·s (s the V scale of the token, or of its
  // group) in two parts: columns c < 8 the high part hi = fp16(P'), columns
  // c >= 8 -- which would otherwise repeat columns c - 8 -- the remainder
  // lo = fp16(P' - hi), each rounded once from the exact product (v_fma_mix),
  // so the two column halves together hold P' to about 2^-22 and are added
  // when the wave's partial is formed.  p_lo = p * lo_sel is p in the lanes
  // c >= 8 and 0 elsewhere: there fp16(p_lo·s) is hi, and every lane's operand
  // is fp16(p·s - that), i.e. hi in columns c < 8 and lo in columns c >= 8.
  // int8 V always takes both parts (three VALU ops per element); 4-bit and
  // affine V, whose P' has four (two) groups per token, only when EXACT
  // (fewer than EXACT_PV_BELOW cached tokens), else every column holds hi,
  // rounded once, and only columns c < 8 are read.
  const float lo_sel = c < 8 ? 0.f : 1.f;
  if constexpr (VB == 8) {
    v8h pb;
#pragma unroll
    for (int idx = 0; idx < 8; ++idx) {
      const uint32_t sw = (uint32_t)vs[idx >> 1];
      const _Float16 sh = __builtin_bit_cast(_Float16, (uint16_t)((idx & 1) ? (sw >> 16) : (sw & 0xffffu)));
      const _Float16 hi = (_Float16)__builtin_fmaf(p[idx] * lo_sel, (float)sh, 0.f);
      pb[idx] = (_Float16)__builtin_fmaf(p[idx], (float)sh, -(float)hi);
    }
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      const v8h a0 = i8x8_to_h8((uint32_t)R.v8[n >> 1][2 * (n & 1)], (uint32_t)R.v8[n >> 1][2 * (n & 1) + 1]);
      st.acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, pb, st.acc[n], 0, 0, 0);
    }
  } else if constexpr (is_a4(VB)) {
    // affine 4-bit V, v = s q + b per 64-dim group: the A operand is q, exact
    // in fp16 (nibble under the fp16 exponent of 1024 or 64, minus that
    // offset), B = P' = p·s per group (high and low parts as above), and
    // Σ p·b per group is kept aside and added to the group's dims at the end.
    // Scales and biases are stored in the nibble unpack's pair order
    // (s4_slot): dword e of a run holds positions (e, e+4).
    const v2h k1024 = {(_Float16)1024.0f, (_Float16)1024.0f}, k64 = {(_Float16)64.0f, (_Float16)64.0f};
    float p_lo[8];
#pragma unroll
    for (int idx = 0; idx < 8; ++idx) p_lo[idx] = p[idx] * lo_sel;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      v8h pb;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t sw = (uint32_t)vs4[g][e], bw = (uint32_t)vz4[g][e];
        constexpr bool F16 = meta_f16(VB);
        const float slo = meta_lo<F16>(sw), shi = meta_hi<F16>(sw);
        const float blo = meta_lo<F16>(bw), bhi = meta_hi<F16>(bw);
        if constexpr (EXACT) {
          const _Float16 h0 = (_Float16)(p_lo[e] * slo), h1 = (_Float16)(p_lo[e + 4] * shi);
          pb[2 * e] = (_Float16)__builtin_fmaf(p[e], slo, -(float)h0);
          pb[2 * e + 1] = (_Float16)__builtin_fmaf(p[e + 4], shi, -(float)h1);
        } else {
          pb[2 * e] = (_Float16)(p[e] * slo);
          pb[2 * e + 1] = (_Float16)(p[e + 4] * shi);
        }
        st.vb[g] = fmaf(p[e], blo, fmaf(p[e + 4], bhi, st.vb[g]));
      }
#pragma unroll
      for (int nn = 0; nn < 4; ++nn) {
        const int n = 4 * g + nn;
        const uint32_t w = (uint32_t)R.v4[n >> 2][n & 3], w8 = w >> 8;
        v8h a;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t t = (e & 1) ? and_or(e < 2 ? w : w8, 0x00f000f0u, 0x54005400u)
                                     : and_or(e < 2 ? w : w8, 0x000f000fu, 0x64006400u);
          const v2h d = __builtin_bit_cast(v2h, t) - ((e & 1) ? k64 : k1024);
          a[2 * e] = d[0];
          a[2 * e + 1] = d[1];
        }
        st.acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb, st.acc[n], 0, 0, 0);
      }
    }
  } else {
    // uint4 V: the A operand is q - z, exact in fp16, and the scale of the
    // (token, group) goes into the B operand, P' = p·s in high and low parts
    // as above, one B operand per 32-dim group.  The nibble unpack yields
    // positions (e, e+4) of the lane's run as one fp16 pair: low nibbles under
    // the fp16 exponent of 1024 read 1024 + q, high nibbles under that of 64
    // read 64 + q.  Scales and zero-points are stored in that pair order
    // (s4_slot), so dword e of a run is the pair for unpack step e; the
    // zero-points arrive here with that step's offset already added (z + 1024
    // or z + 64, exact: z is a small integer), so one subtraction gives q - z.
    float p_lo[8];
#pragma unroll
    for (int idx = 0; idx < 8; ++idx) p_lo[idx] = p[idx] * lo_sel;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      v8h pb;
      v2h zq[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // copies first: a bit_cast of a vector subscript reads element 0
        const uint32_t sw = (uint32_t)vs4[g][e], zw = (uint32_t)vz4[g][e];
        const v2h sv = __builtin_bit_cast(v2h, sw);
        // fmas on an fp16 scale lower to v_fma_mix*, which read the fp16
        // operand directly (a plain multiply costs a conversion per scale)
        if constexpr (EXACT) {
          const _Float16 h0 = (_Float16)__builtin_fmaf(p_lo[e], (float)sv[0], 0.f);
          const _Float16 h1 = (_Float16)__builtin_fmaf(p_lo[e + 4], (float)sv[1], 0.f);
          pb[2 * e] = (_Float16)__builtin_fmaf(p[e], (float)sv[0], -(float)h0);
          pb[2 * e + 1] = (_Float16)__builtin_fmaf(p[e + 4], (float)sv[1], -(float)h1);
        } else {
          // p·s rounded to fp16 once, into the two halves of one register
          uint32_t w2;
          asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel_hi:[0,1,0]" : "=v"(w2) : "v"(p[e]), "v"(sw));
          asm("v_fma_mixhi_f16 %0, %1, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "+v"(w2) : "v"(p[e + 4]), "v"(sw));
          const v2h pp = __builtin_bit_cast(v2h, w2);
          pb[2 * e] = pp[0];
          pb[2 * e + 1] = pp[1];
        }
        zq[e] = __builtin_bit_cast(v2h, zw);  // z plus the unpack offset, added at the LDS hand-out
      }
#pragma unroll
      for (int nn = 0; nn < 2; ++nn) {
        const int n = 2 * g + nn;
        const uint32_t w = (uint32_t)R.v4[n >> 2][n & 3], w8 = w >> 8;
        v8h a;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t t = (e & 1) ? and_or(e < 2 ? w : w8, 0x00f000f0u, 0x54005400u)
                                     : and_or(e < 2 ? w : w8, 0x000f000fu, 0x64006400u);
          const v2h d = __builtin_bit_cast(v2h, t) - zq[e];
          a[2 * e] = d[0];
          a[2 * e + 1] = d[1];
        }
        st.acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb, st.acc[n], 0, 0, 0);
      }
    }
  }
}

// Chunk buffers per wave: two (one chunk in flight while one is computed).
// Measured against three on MI355X: 13% faster at 32K int8 tokens, 2% at
// 252K, 7% for the affine format at 32K, even for uint4 at 131K.
template <int KB, int VB>
struct Depth {
  static constexpr int value = 2;
};

template <int KB, int VB, int WAVES, bool EXACT, bool MASK>
__global__ __launch_bounds__(64 * WAVES) void decode_kernel(const DecodeArgs a) {
  using LD = Lds<WAVES>;
  __shared__ __attribute__((aligned(16))) char smem[LD::bytes];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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

  constexpr int64_t KROW = KB == 8 || is_a8(KB) ? HEAD_DIM : HEAD_DIM / 2;  // code bytes per token
  constexpr int64_t VROW = VB == 8 ? HEAD_DIM : HEAD_DIM / 2;
  constexpr int64_t KSROW = KB == 8 ? 1 : 4;                   // fp16 scales per token
  constexpr int64_t VSROW = VB == 8 ? 1 : 4;
  Res R;
  R.k = make_rsrc((const int8_t*)a.kq + bh * cap * KROW, cap * KROW);
  R.v = make_rsrc((const int8_t*)a.vq + bh * cap * VROW, cap * VROW);
  R.ks = make_rsrc(a.ks + bh * cap * KSROW, cap * KSROW * 2);
  R.vs = make_rsrc(a.vs + bh * cap * VSROW, cap * VSROW * 2);
  R.kz = KB == 4 ? make_rsrc(a.kz + bh * cap * 4, cap * 8) : R.ks;
  R.vz = VB == 4 ? make_rsrc(a.vz + bh * cap * 4, cap * 8) : R.vs;
  R.none = make_rsrc(a.ks, 0);

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
        append_v4_pair<is_a4(VB), meta_f16(VB)>(a.vnew, b, h, odd ? -1 : 0, !odd, odd, (uint8_t*)a.vq, (uint16_t*)a.vs,
                                     (uint16_t*)a.vz, bh, cap, pos & ~(int64_t)1, lane);
      }
    }
    __threadfence_block();
    __syncthreads();
  }

  // The query rows are loaded first: everything below overlaps their latency.
  const int hh = tid >> 5, d0 = (tid & 31) * 4;
  const int hq_ld = h * a.G + (hh < a.G ? hh : 0);
  const v4i qraw = load_q_raw(a.q, (int64_t)b * a.q_sb + (int64_t)hq_ld * a.q_sh + d0, a.q_dtype);

  // Wave w takes chunks w, w+4, ... of the split; a ring of NBUF chunk buffers
  // keeps NBUF-1 chunks in flight while one is computed.  Slots past the
  // wave's last chunk load nothing (NO_CHUNK) but are still issued.
  constexpr int NBUF = Depth<KB, VB>::value;
  const int n_split = (t_end - t_begin + CH - 1) / CH;
  const int n_w = n_split > wave ? (n_split - wave + WAVES - 1) / WAVES : 0;
  const int blk0 = t_begin / CH + wave;
  const LaneOff lo = lane_offsets<KB, VB>(lane);
  const char* mbase = nullptr;  // uint4 K and V: this lane's metadata array and offset
  if constexpr (KB == 4 && VB == 4) {
    const int sel = lane >> 4;
    const uint16_t* arr = sel == 0 ? a.ks : sel == 1 ? a.kz : sel == 2 ? a.vs : a.vz;
    mbase = (const char*)arr + bh * cap * 8 + (lane & 15) * 16;
  }
  Chunk buf[NBUF];
#pragma unroll
  for (int i = 0; i < NBUF - 1; ++i) load_chunk<KB, VB>(buf[i], R, lo, i < n_w, blk0 + WAVES * i, mbase);
  // MASK: the bias row of this lane's head (column c, head c mod 8), two
  // 16-byte runs per chunk, loaded with the chunk into a ring of its own
  v4i bz[NBUF][2];
  __amdgpu_buffer_rsrc_t rb = R.none;
  uint32_t boff = 0;
  if constexpr (MASK) {
    const int64_t base = (int64_t)b * a.bias.sb + (int64_t)h * a.bias.skv;
    rb = make_rsrc(a.bias.p + base, (a.bias.extent - base) * 4);
    const int gq = (c & 7) < a.G ? (c & 7) : 0;
    boff = (uint32_t)(((int64_t)gq * a.bias.sg + 4 * kg) * 4);
  }
  const auto load_bias = [&](v4i(&z)[2], bool ok, int blk) {
    if constexpr (MASK) {
      const __amdgpu_buffer_rsrc_t r = ok ? rb : R.none;
      const uint32_t t0 = (uint32_t)blk * CH * 4;
      z[0] = ld128<0>(r, boff + t0, 0);
      z[1] = ld128<0>(r, boff + t0 + 64, 0);
    }
  };
#pragma unroll
  for (int i = 0; i < NBUF - 1; ++i) load_bias(bz[i], i < n_w, blk0 + WAVES * i);

  // Quantize the query into MFMA operands while the chunks stream in.
  {
    float x[4];
    q_raw_to_float(qraw, a.q_dtype, x);
    const float mul = hh < a.G ? a.q_mul : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] *= mul;
    prepare_query<KB, 64 * WAVES>(x, smem, tid);
  }
  __syncthreads();

  constexpr int NOP = KB == 8 || is_a8(KB) ? 2 : 4;
  v4i qop[NOP];
#pragma unroll
  for (int o = 0; o < NOP; ++o) qop[o] = ((const v4i*)(smem + LDS_QOP))[o * 64 + lane];
  // query quantization step of this lane's head; an all-zero query has step 0
  // and all-zero scores, for which any positive step is exact
  const float qsc_h = ((const float*)(smem + LDS_QSC))[c & 7];
  const float qsc = qsc_h > 0.f ? qsc_h : 1.f;
  const float bmul = MASK ? LOG2E / qsc : 0.f;
  // query sums per group of this lane's head (exact integers): int4 K, the
  // lane's two 32-dim groups; affine K, the two 64-dim groups
  float qsum_a = 0.f, qsum_b = 0.f;
  if constexpr (KB == 4) {
    const int* qsum = (const int*)(smem + LDS_QSUM);
    qsum_a = (float)qsum[(c & 7) * 4 + (c >> 3)];
    qsum_b = (float)qsum[(c & 7) * 4 + 2 + (c >> 3)];
  } else if constexpr (is_a8(KB)) {
    const int* qsum = (const int*)(smem + LDS_QSUM);
    qsum_a = (float)(qsum[(c & 7) * 4] + qsum[(c & 7) * 4 + 1]);
    qsum_b = (float)(qsum[(c & 7) * 4 + 2] + qsum[(c & 7) * 4 + 3]);
  }

  State st;
  st.m = NEG_INF;
  st.l = 0.f;
#pragma unroll
  for (int n = 0; n < 8; ++n) st.acc[n] = (v4f){0.f, 0.f, 0.f, 0.f};
  st.vb[0] = st.vb[1] = 0.f;

  // Step i loads chunk i+NBUF-1 into the buffer freed by step i-1, then
  // computes chunk i.  The ring is unrolled so buffer indices are static, and
  // the step count is padded to a whole number of revolutions: every step
  // issues its loads (padding steps through the empty resource), only the
  // compute of padding steps is skipped, and the loop has a single back edge.
  // The compiler then counts the loads in flight exactly on every path.
  const int n_pad = (n_w + NBUF - 1) / NBUF * NBUF;
  for (int i0 = 0; i0 < n_pad; i0 += NBUF) {
#pragma unroll
    for (int j = 0; j < NBUF; ++j) {
      const int i = i0 + j;
      load_chunk<KB, VB>(buf[(j + NBUF - 1) % NBUF], R, lo, i + NBUF - 1 < n_w, blk0 + WAVES * (i + NBUF - 1),
                         mbase);
      load_bias(bz[(j + NBUF - 1) % NBUF], i + NBUF - 1 < n_w, blk0 + WAVES * (i + NBUF - 1));
      if (i < n_w)
        process_chunk<KB, VB, EXACT, MASK>(buf[j], st, qop, qsc, qsum_a, qsum_b, t_end - (blk0 + WAVES * i) * CH,
                                           lane, smem + LD::meta + wave * 1024, bz[j], bmul);
    }
  }

  // ---------------- wave partial -> LDS ----------------
  st.l = sum_xor32(sum_xor16(st.l));
  // the P·V sums of the high (columns c < 8) and low (c + 8) parts of P'
  if constexpr (VB == 8 || EXACT) {
#pragma unroll
    for (int n = 0; n < 8; ++n)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float x = st.acc[n][i];  // copy first: a bit_cast of a vector subscript reads element 0
        st.acc[n][i] = x + dpp_ror8f(x);
      }
  }
  if constexpr (is_a4(VB)) {  // the bias terms join every dim of their group
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      float vb = st.vb[g];
      vb = sum_xor32(sum_xor16(vb));
#pragma unroll
      for (int nn = 0; nn < 4; ++nn) st.acc[4 * g + nn] += vb;
    }
  }
  float* part = (float*)(smem + LD::part);
  float* pstat = (float*)(smem + LD::pstat);
  if (c < 8 && c < a.G) {
#pragma unroll
    for (int n = 0; n < 8; ++n)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        part[(wave * 8 + c) * PART_ROW + 16 * n + 4 * kg + i] = st.acc[n][i];
      }
    if (kg == 0) {
      pstat[(wave * 8 + c) * 2 + 0] = st.m;
      pstat[(wave * 8 + c) * 2 + 1] = st.l;
    }
  }
  __syncthreads();

  // ---------------- workgroup partial (or the output when S == 1) ----------------
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
      acc4 += f * *(const v4f*)(part + (w * 8 + hh) * PART_ROW + d0);
      l += f * pstat[(w * 8 + hh) * 2 + 1];
    }
    if (a.S == 1) {
      if (sink != NEG_INF) l += __builtin_amdgcn_exp2f(sink - M);
      const v4f o = l > 0.f ? acc4 / l : acc4;
      store_out4(a.out, ((int64_t)b * a.Hq + h * a.G + hh) * HEAD_DIM + d0, o, a.out_dtype);
    } else {
      const int64_t row = (bh * a.S + split) * 8 + hh;
      *(v4f*)(a.ws_acc + row * HEAD_DIM + d0) = acc4;
      if ((tid & 31) == 0) *(v2f*)(a.ws_stat + row * 2) = (v2f){M, l};
    }
  }
}

// Cross-split merge (megakernel.py:276-318).  One wavefront per (query head,
// quarter of the dims, batch): lane (sg, d4) sums splits sg, sg+8, ... for
// dims 32*quarter + 4*d4 .. +3, and lane l also owns the (m, l) statistics of
// splits l, l+64, ...  Every load (partials, statistics, sink) is issued at
// entry as an unconditional buffer load (slots past the last split read zeros)
// and the reductions stay inside the wavefront, so the kernel makes a single
// trip to memory.
template <int PER>  // splits per lane group: S <= 8 * PER
__global__ __launch_bounds__(64) void decode_merge_kernel(const DecodeArgs a) {
  __shared__ float wts[8 * PER];
  constexpr int SPL = (8 * PER + 63) / 64;  // statistics slots per lane
  const int lane = threadIdx.x, d4 = lane & 7, sg = lane >> 3;
  const int hq = blockIdx.x >> 2, qd = blockIdx.x & 3, b = blockIdx.y;
  const int h = hq / a.G, hh = hq - h * a.G;
  const int64_t bh = (int64_t)b * a.Hkv + h;
  const int S = a.S;
  // partials of this (b, h): [S][8][128] floats and [S][8][2] statistics
  const __amdgpu_buffer_rsrc_t racc = make_rsrc(a.ws_acc + bh * S * 8 * HEAD_DIM, (int64_t)S * 8 * HEAD_DIM * 4);
  const __amdgpu_buffer_rsrc_t rst = make_rsrc(a.ws_stat + bh * S * 8 * 2, (int64_t)S * 8 * 2 * 4);
  const uint32_t voff = (uint32_t)((hh * HEAD_DIM + 32 * qd + 4 * d4) * 4);
  v4f v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i)  // whole offset in voffset: it is range-checked (soffset may not be)
    v[i] = __builtin_bit_cast(v4f, ld128<0>(racc, voff + (uint32_t)(sg + 8 * i) * 8 * HEAD_DIM * 4, 0));
  v2i stw[SPL];
#pragma unroll
  for (int k = 0; k < SPL; ++k) stw[k] = ld64<0>(rst, (uint32_t)(((lane + 64 * k) * 8 + hh) * 8), 0);
  // the sink logit through a buffer too (no sinks: an empty resource reads 0),
  // so it joins the same batch of loads instead of a scalar load waited on first
  const bool has_sink = a.sinks != nullptr;
  const __amdgpu_buffer_rsrc_t rsk = make_rsrc(has_sink ? a.sinks : a.ws_stat, has_sink ? a.Hq * 4 : 0);
  const uint32_t sink_bits = ld32<0>(rsk, (uint32_t)hq * 4, 0);

  float ms[SPL], ls[SPL], M = NEG_INF;
#pragma unroll
  for (int k = 0; k < SPL; ++k) {
    const int m_bits = stw[k][0], l_bits = stw[k][1];  // copies: bit_cast of a vector subscript reads lane 0
    const bool ok = lane + 64 * k < S;
    ms[k] = ok ? __builtin_bit_cast(float, m_bits) : NEG_INF;
    ls[k] = ok ? __builtin_bit_cast(float, l_bits) : 0.f;
    M = maxp(M, ms[k]);
  }
  const float sink = has_sink ? __builtin_bit_cast(float, sink_bits) * LOG2E : NEG_INF;
  M = fmaxf(wave_max(M), sink);
  float lw = 0.f;
#pragma unroll
  for (int k = 0; k < SPL; ++k) {
    const float w = (ms[k] == NEG_INF || M == NEG_INF) ? 0.f : __builtin_amdgcn_exp2f(ms[k] - M);
    lw += w * ls[k];
    if (lane + 64 * k < 8 * PER) wts[lane + 64 * k] = w;
  }
  lw = wave_sum(lw);
  __syncthreads();
  v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < PER; ++i) acc += wts[sg + 8 * i] * v[i];
  // sum over the eight split groups sg (lanes d4 + 8 sg): xor 8, 16, 32
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float t = acc[e];
    t += dpp_f<DPP_ROR8>(t);
    acc[e] = sum_xor32(sum_xor16(t));
  }
  if (sg == 0) {
    const float L = sink != NEG_INF ? lw + __builtin_amdgcn_exp2f(sink - M) : lw;
    const v4f o = L > 0.f ? acc * (1.f / L) : acc;
    store_out4(a.out, ((int64_t)b * a.Hq + hq) * HEAD_DIM + 32 * qd + 4 * d4, o, a.out_dtype);
  }
}

template <int KB, int VB, int W, bool EXACT>
static void launch_partial(const DecodeArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((decode_kernel<KB, VB, W, EXACT, false>), dim3(a.S, a.Hkv, a.B), dim3(64 * W), 0, stream, a);
}

template <int KB, int VB, int W>
static void launch_partial_pv(const DecodeArgs& a, hipStream_t stream) {
  if (a.T < EXACT_PV_BELOW) launch_partial<KB, VB, W, true>(a, stream);
  else launch_partial<KB, VB, W, false>(a, stream);
}

// A bias (mask array) may leave any row a few visible keys: the exact P·V,
// four waves, every format.
template <int KB, int VB>
static void launch_masked(const DecodeArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((decode_kernel<KB, VB, 4, true, true>), dim3(a.S, a.Hkv, a.B), dim3(256), 0, stream, a);
}

hipError_t launch_decode_partial(int kb, int vb, const DecodeArgs& a, hipStream_t stream) {
  if (a.bias.p != nullptr) {
    if (kb == 8 && vb == 8) launch_masked<8, 8>(a, stream);
    else if (kb == 8 && vb == 4) launch_masked<8, 4>(a, stream);
    else if (kb == 4 && vb == 8) launch_masked<4, 8>(a, stream);
    else if (kb == 4 && vb == 4) launch_masked<4, 4>(a, stream);
    else if (kb == FMT_A8) launch_masked<FMT_A8, FMT_A4>(a, stream);
    else launch_masked<FMT_A8H, FMT_A4H>(a, stream);
    return hipGetLastError();
  }
  if (kb == 8 && vb == 8) launch_partial<8, 8, 4, true>(a, stream);
  else if (kb == 8 && vb == 4) launch_partial_pv<8, 4, 4>(a, stream);
  else if (kb == 4 && vb == 8) launch_partial<4, 8, 4, true>(a, stream);
  else if (kb == FMT_A8 && vb == FMT_A4) launch_partial_pv<FMT_A8, FMT_A4, 4>(a, stream);
  else if (kb == FMT_A8H && vb == FMT_A4H) launch_partial_pv<FMT_A8H, FMT_A4H, 4>(a, stream);
  else if (a.span / CH >= UINT4_WIDE_CHUNKS) launch_partial_pv<4, 4, 8>(a, stream);
  else launch_partial_pv<4, 4, 4>(a, stream);
  return hipGetLastError();
}

hipError_t launch_decode_merge(const DecodeArgs& a, hipStream_t stream) {
  if (a.S == 1) return hipSuccess;  // the partial kernel wrote the output
  const dim3 grid(a.Hq * 4, a.B), block(64);
  if (a.S <= 8) hipLaunchKernelGGL(decode_merge_kernel<1>, grid, block, 0, stream, a);
  else if (a.S <= 16) hipLaunchKernelGGL(decode_merge_kernel<2>, grid, block, 0, stream, a);
  else if (a.S <= 32) hipLaunchKernelGGL(decode_merge_kernel<4>, grid, block, 0, stream, a);
  else if (a.S <= 64) hipLaunchKernelGGL(decode_merge_kernel<8>, grid, block, 0, stream, a);
  else if (a.S <= 128) hipLaunchKernelGGL(decode_merge_kernel<16>, grid, block, 0, stream, a);
  else hipLaunchKernelGGL(decode_merge_kernel<32>, grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace rec
