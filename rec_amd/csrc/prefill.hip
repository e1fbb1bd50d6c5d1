// Chunked prefill attention over the int8 KV cache on bf16 / fp16 matrix cores
// (gfx950).
//
// Restates the prefill branch of Attention.__call__
// (engine/src/rec_mlx/model.py:191-203): the new tokens were quantize-appended
// first (model.py:177-178), then the L new queries attend over the whole
// cache, the new tokens included, with the causal "string" mask of
// model.py:122-125 (query i sits at position T-L+i) and the per-head sink
// logit in the softmax denominator.  The reference dequantizes the cache to the
// query dtype; here K/V codes are converted to bf16/fp16 exactly (|q| <= 127)
// and the row scales are applied outside the matrix products: the K scale to
// the scores, the V scale folded into the probabilities before their one
// rounding.  Q·K^T runs on bf16 MFMAs for bf16 queries (fp16 for fp16
// queries); P·V always on fp16 MFMAs, whose 11-bit significand keeps the
// rounded probabilities within 2^-12 (bf16 would allow 2^-9, more than the
// 1e-3 output tolerance when one token dominates).
//
// Work decomposition.  Grid (ceil(L/32), Hkv, B), 512 threads = 8 wavefronts;
// wave w owns query head w of the KV head's GQA group and 32 query positions.
// Each 128-token K/V tile is loaded once per workgroup, converted into
// double-buffered LDS (149 KB) and shared by the 8 waves, which compute it in
// four 32-token units, software-pipelined so that one unit's Q·Kᵀ runs on the
// matrix cores while the previous unit's softmax runs on the VALU.  A grid too
// small to fill the chip (a short chunk over a long cache) splits the keys:
// grid x = query blocks x splits, each workgroup writes an unnormalised
// partial, and prefill_merge_kernel combines the splits as the decode's merge
// does (megakernel.py:276-318).
//
// S^T = K Q^T on 16x16x32 MFMAs (A = 16 tokens x 32 dims from LDS, B = Q^T held
// in registers), which leaves lane (c, g) with the scores of query row c for
// tokens 16j + 4g + i -- the order the cache keeps V in inside a 32-token
// block.  P·V then takes A = V^T straight from LDS (dims x tokens, cache
// order) and B = P'^T from the lane's own registers.
#include <algorithm>

#include "kernels.h"

namespace rec {

constexpr int PF_QB = 32;           // query positions per workgroup
constexpr int PF_KROW = 144;        // LDS row pitch of K (elements): 128 + 16 pad

// Tile geometry per cache format: tokens per K/V tile in LDS (one barrier per
// tile) and the LDS row pitch of V (positions + 16 pad).  A bf16 cache moves
// twice the bytes per token, so its tiles are half as long (same registers).
template <bool KVB>
struct PfTile {
  static constexpr int KT = KVB ? 64 : 128;
  static constexpr int VROW = KT + 16;
  static constexpr int K_ELEMS = KT * PF_KROW;
  static constexpr int V_ELEMS = HEAD_DIM * VROW;
};

template <bool BF16>
struct MT;
template <>
struct MT<true> {
  typedef v8bf vec;
  typedef __bf16 elem;
  static __device__ __forceinline__ v4f mfma(vec a, vec b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  // exact for integers |x| <= 256 and for bf16 inputs; round-to-nearest-even otherwise
  static __device__ __forceinline__ elem from_float(float x) { return (__bf16)x; }
};
template <>
struct MT<false> {
  typedef v8h vec;
  typedef _Float16 elem;
  static __device__ __forceinline__ v4f mfma(vec a, vec b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ elem from_float(float x) { return (_Float16)x; }
};

// One thread's share of a 128-token tile as loaded from HBM: 16 bytes of K
// and of V from each of two cache blocks, and one fp16 scale (threads 0..255:
// 128 K scales then 128 V scales).
struct TileRegs {
  v4i k[2], v[2];
  uint32_t s;
};

__device__ __forceinline__ void load_tile(TileRegs& R, const PrefillArgs& a, int64_t bh, int t0, int tid, int t_end) {
  const int o = (tid & 255) * 16;  // byte in block
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    const int bk = 2 * part + (tid >> 8);  // cache block within the tile
    const int blk = (t0 >> 5) + bk;
    const bool live = t0 + 32 * bk < t_end;
    const int8_t* kb = (const int8_t*)a.kq + (bh * (a.cap / BLOCK_T) + blk) * 4096;
    const int8_t* vb = (const int8_t*)a.vq + (bh * (a.cap / BLOCK_T) + blk) * 4096;
    R.k[part] = live ? __builtin_nontemporal_load((const v4i*)(kb + o)) : (v4i){0, 0, 0, 0};
    R.v[part] = live ? __builtin_nontemporal_load((const v4i*)(vb + o)) : (v4i){0, 0, 0, 0};
  }
  R.s = 0;
  if (tid < 256) {
    const int which = tid >> 7, tt = tid & 127;  // 0 = K scale, 1 = V scale
    const uint16_t* sp = which == 0 ? a.ks : a.vs;
    if (t0 + tt < t_end) R.s = sp[(bh * (a.cap / BLOCK_T) + (t0 >> 5) + (tt >> 5)) * 32 + block_pos(tt & 31)];
  }
}

template <bool BF16>
__device__ __forceinline__ void store_tile(const TileRegs& R, typename MT<BF16>::elem* Kl, _Float16* Vl, float* KS,
                                           float* VS, int tid, float q_mul) {
  typedef typename MT<BF16>::elem E;
  const int o = (tid & 255) * 16;
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    const int bk = 2 * part + (tid >> 8);
    // K block: [2 halves][32 tokens][64 B] -> LDS [token][dim]
    {
      const int m = o >> 11, r = (o & 2047) >> 6, e0 = o & 63;
      E* dst = Kl + (32 * bk + r) * PF_KROW + 64 * m + e0;
#pragma unroll
      for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int b = 0; b < 4; ++b)
          dst[4 * w + b] = MT<BF16>::from_float((float)(int8_t)((uint32_t)R.k[part][w] >> (8 * b)));
    }
    // V block: 16-byte run o = [n/2][c][position group pg] holds positions
    // 8pg .. 8pg+7 of dims 16n + c for n = 2(o/1024) and that + 1 -> LDS
    // [dim][128 positions of the tile]
    {
      const int n0 = 2 * (o >> 10), cc = (o >> 6) & 15, pg = (o >> 4) & 3;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        _Float16* dst = Vl + (16 * (n0 + half) + cc) * PfTile<false>::VROW + 32 * bk + 8 * pg;
#pragma unroll
        for (int w = 0; w < 2; ++w)
#pragma unroll
          for (int b = 0; b < 4; ++b)
            dst[4 * w + b] = (_Float16)(float)(int8_t)((uint32_t)R.v[part][2 * half + w] >> (8 * b));
      }
    }
  }
  // K scales carry the softmax scale (log2 domain)
  if (tid < 256) (tid < 128 ? KS : VS)[tid & 127] = half_bits_to_float(R.s) * (tid < 128 ? q_mul : 1.f);
}

// bf16 cache: a 64-token tile is 16 KB of K and of V; thread tid takes the
// 16-byte chunks tid and tid + 512 of each, chunk = (token, 8 dims).
__device__ __forceinline__ void load_tile_bf16(TileRegs& R, const PrefillArgs& a, int b, int h, int t0, int tid,
                                               int t_end) {
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    const int id = part * 512 + tid, tok = id >> 4, d0 = (id & 15) * 8;
    const bool live = t0 + tok < t_end;
    const int64_t row = (int64_t)(t0 + tok) * HEAD_DIM + d0;
    const uint16_t* kp = (const uint16_t*)a.kq + (int64_t)b * a.k_sb + (int64_t)h * a.k_sh + row;
    const uint16_t* vp = (const uint16_t*)a.vq + (int64_t)b * a.v_sb + (int64_t)h * a.v_sh + row;
    R.k[part] = live ? __builtin_nontemporal_load((const v4i*)kp) : (v4i){0, 0, 0, 0};
    R.v[part] = live ? __builtin_nontemporal_load((const v4i*)vp) : (v4i){0, 0, 0, 0};
  }
}

// K rows as they are (bf16 queries) or in fp16; V transposed into [dim][cache
// position] as fp16 (exact for bf16 values in fp16's normal range), the
// position of token t of a 32-token unit being block_pos(t) as in the int8
// layout; the "scales" are the softmax scale and 1.
template <bool BF16>
__device__ __forceinline__ void store_tile_bf16(const TileRegs& R, typename MT<BF16>::elem* Kl, _Float16* Vl,
                                                float* KS, float* VS, int tid, float q_mul) {
  constexpr int VROW = PfTile<true>::VROW;
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    const int id = part * 512 + tid, tok = id >> 4, d0 = (id & 15) * 8;
    if constexpr (BF16) {
      *(v4i*)(Kl + tok * PF_KROW + d0) = R.k[part];
    } else {
      v8h kh;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t w = (uint32_t)R.k[part][e];
        kh[2 * e] = (_Float16)__builtin_bit_cast(float, w << 16);
        kh[2 * e + 1] = (_Float16)__builtin_bit_cast(float, w & 0xffff0000u);
      }
      *(v8h*)(Kl + tok * PF_KROW + d0) = kh;
    }
    const int col = (tok & ~31) + block_pos(tok & 31);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t w = (uint32_t)R.v[part][e];
      Vl[(d0 + 2 * e) * VROW + col] = (_Float16)__builtin_bit_cast(float, w << 16);
      Vl[(d0 + 2 * e + 1) * VROW + col] = (_Float16)__builtin_bit_cast(float, w & 0xffff0000u);
    }
  }
  if (tid < 2 * PfTile<true>::KT) (tid < PfTile<true>::KT ? KS : VS)[tid & (PfTile<true>::KT - 1)] = tid < PfTile<true>::KT ? q_mul : 1.f;
}

// S^T = K Q^T for one 32-token unit of one wave: 32 query rows (two column
// tiles of 16) of one head; lane (c, g) receives the scores of query row c for
// tokens 16j + 4g + i of the unit.
template <bool BF16>
__device__ __forceinline__ void qk_unit(const typename MT<BF16>::elem* K, const typename MT<BF16>::vec (&qop)[2][4],
                                        v4f (&s4)[2][2], int c, int g) {
  typedef typename MT<BF16>::vec V8;
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int j = 0; j < 2; ++j) s4[rt][j] = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const V8 ka = *(const V8*)(K + (16 * j + c) * PF_KROW + 32 * ks + 8 * g);
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) s4[rt][j] = MT<BF16>::mfma(ka, qop[rt][ks], s4[rt][j]);
    }
}

// Softmax of one unit's scores, then O^T += V^T P'^T.  mask: some token of the
// unit lies past the cache end or past a query's causal diagonal (only units
// that reach a query block's diagonal); one loop under one uniform branch.
//
// Row state (per query row rt of the lane): m_use, the offset the
// probabilities are taken against (log2 domain; 0 before the row's first
// finite score), thr, the bound past which a score moves it (-inf until the
// row has seen a finite score, then RESCALE_GAP), and l_run, the sum of
// probabilities.  t = s * ksc - m_use is one fma per score.
template <int VROW, bool EXACT>
__device__ __forceinline__ void softmax_pv_unit(const v4f (&s4)[2][2], const _Float16* Vv, const float* KS,
                                                const float* VS, float (&m_use)[2], float (&thr)[2],
                                                float (&l_run)[2], v4f (&acc)[8][2], int t0, int t_end, int qabs0,
                                                int causal, int window, bool mask, int c, int g) {
  v8h pb[2], pl[2];  // P'^T: high parts, and (EXACT) the remainders
  // Range: P' = p·s feeds an fp16 operand, finite while p·s < 65504.  A V
  // scale of 2 or more among the lane's tokens (fp32 exponent bit 30;
  // |v| >= 254) makes its bound 0 for this unit, so its p <= 1 and
  // P' <= s <= 65504.
  bool big;
  {
    const v4i w0 = *(const v4i*)(&VS[4 * g]), w1 = *(const v4i*)(&VS[16 + 4 * g]);
    const v4i o = w0 | w1;
    big = ((uint32_t)(o[0] | o[1] | o[2] | o[3]) & 0x40000000u) != 0;
  }
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    // scale (K scale x softmax scale) and offset in one fma, mask, online
    // softmax per query row (lane column c of tile rt)
    float t[8];
    const int qabs = qabs0 + 16 * rt + c;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const v4f ksc = *(const v4f*)(&KS[16 * j + 4 * g]);
#pragma unroll
      for (int i = 0; i < 4; ++i) t[4 * j + i] = __builtin_fmaf(s4[rt][j][i], ksc[i], -m_use[rt]);
    }
    if (mask) {
      // first and last visible token of this row, relative to the lane's first token t0 + 4g
      const int last = (causal ? min(qabs, t_end - 1) : t_end - 1) - t0 - 4 * g;
      const int first = window > 0 ? qabs - window + 1 - t0 - 4 * g : INT32_MIN;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int pos = 16 * (k >> 2) + (k & 3);
        if (pos > last || pos < first) t[k] = NEG_INF;
      }
    }
    float cmax = t[0];
#pragma unroll
    for (int k = 1; k < 8; ++k) cmax = maxp(cmax, t[k]);
    // The offset moves only when a score passes it by more than RESCALE_GAP
    // (log2 units): until then probabilities up to 2^RESCALE_GAP are as exact
    // in fp16 P' and the fp32 sums as ones up to 1, and the rescale (a
    // cross-lane max, an exp and 32 multiplies per row tile) runs far less
    // often (measured 2% faster).  A row's max passes the bound iff one of its
    // four lanes' maxima does.
    if (__ballot(cmax > (big ? fminf(thr[rt], 0.f) : thr[rt]))) {
      cmax = max_xor32(max_xor16(cmax));  // the row's max of t
      // a row with finite scores so far moves to max(offset, row max); a new
      // row takes its first finite max; an all-masked row stays
      float delta = maxp(cmax, thr[rt] == NEG_INF ? cmax : 0.f);
      delta = delta == NEG_INF ? 0.f : delta;
      // a new row's sums are still zero; its delta may be far below zero, where
      // exp2(-delta) would overflow
      const float factor = thr[rt] == NEG_INF ? 0.f : __builtin_amdgcn_exp2f(-delta);
      l_run[rt] *= factor;
#pragma unroll
      for (int n = 0; n < 8; ++n) acc[n][rt] *= factor;
      m_use[rt] += delta;
      thr[rt] = cmax == NEG_INF ? thr[rt] : RESCALE_GAP;
#pragma unroll
      for (int k = 0; k < 8; ++k) t[k] -= delta;
    }
    float lsum = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const v4f vsc = *(const v4f*)(&VS[16 * j + 4 * g]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __builtin_amdgcn_exp2f(t[4 * j + i]);
        lsum += p;
        // B operand of P·V: k index 8g + 4j + i = cache position of token 16j + 4g + i
        const _Float16 hi = (_Float16)(p * vsc[i]);
        pb[rt][4 * j + i] = hi;
        if constexpr (EXACT) pl[rt][4 * j + i] = (_Float16)__builtin_fmaf(p, vsc[i], -(float)hi);
      }
    }
    l_run[rt] += lsum;
  }
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    const v8h va = *(const v8h*)(Vv + (16 * n + c) * VROW + 8 * g);
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      acc[n][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[rt], acc[n][rt], 0, 0, 0);
      if constexpr (EXACT) acc[n][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl[rt], acc[n][rt], 0, 0, 0);
    }
  }
}

template <bool BF16, bool KVB, bool EXACT>
__global__ __launch_bounds__(512) void prefill_kernel(const PrefillArgs a) {
  typedef typename MT<BF16>::elem E;
  typedef typename MT<BF16>::vec V8;
  constexpr int PF_KT = PfTile<KVB>::KT, VROW = PfTile<KVB>::VROW;
  __shared__ __attribute__((aligned(16))) E Kl[2][PfTile<KVB>::K_ELEMS];
  __shared__ __attribute__((aligned(16))) _Float16 Vl[2][PfTile<KVB>::V_ELEMS];
  __shared__ __attribute__((aligned(16))) float KS[2][PF_KT];
  __shared__ __attribute__((aligned(16))) float VS[2][PF_KT];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c = lane & 15, g = lane >> 4;
  // uniform, kept in scalar registers (the division would otherwise leave
  // them, and everything derived from them, in vector registers)
  const int split = __builtin_amdgcn_readfirstlane((int)blockIdx.x / a.nqb);
  const int qb = __builtin_amdgcn_readfirstlane((int)blockIdx.x - split * a.nqb);
  const int q0 = qb * PF_QB, h = blockIdx.y, b = blockIdx.z;
  const int64_t bh = (int64_t)b * a.Hkv + h;
  const int P = (int)(a.T - a.L);  // cached tokens before the new ones
  const int t_blk = a.causal ? min((int)a.T, P + q0 + PF_QB) : (int)a.T;  // the block's keys end here
  const bool active = w < a.G;
  const int hq = h * a.G + (active ? w : 0);

  // Q^T operands: column tile rt holds query rows q0+16rt .. +15, k-step ks dims 32ks..32ks+31.
  V8 qop[2][4];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int qr = min(q0 + 16 * rt + c, a.L - 1);
    const int64_t base = (int64_t)b * a.q_sb + (int64_t)hq * a.q_sh + (int64_t)qr * a.q_st;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) qop[rt][ks][e] = MT<BF16>::from_float(load_as_float(a.q, base + 32 * ks + 8 * g + e, a.q_dtype));
  }

  float m_use[2] = {0.f, 0.f}, thr[2] = {NEG_INF, NEG_INF}, l_run[2] = {0.f, 0.f};
  v4f acc[8][2];
#pragma unroll
  for (int n = 0; n < 8; ++n)
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) acc[n][rt] = (v4f){0.f, 0.f, 0.f, 0.f};

  // a sliding window (bf16 caches only) starts the scan at the first query's first visible key
  const int window = KVB ? a.window : 0;
  const int t_first = window > 0 ? max(0, P + q0 - window + 1) / PF_KT * PF_KT : 0;
  // this workgroup's share of the keys, [lo, t_end): the split's range
  // (tile-aligned) within the query block's [t_first, t_blk); empty for some
  // splits.  A split that ends before t_blk ends on a tile boundary, so its
  // tiles are whole and t_end serves every load, mask and liveness test.
  const int64_t s_lo = a.split_lo + (int64_t)split * a.split_len;
  const int lo = __builtin_amdgcn_readfirstlane((int)max((int64_t)t_first, s_lo));
  const int t_end = __builtin_amdgcn_readfirstlane((int)min((int64_t)t_blk, s_lo + a.split_len));
  const auto fetch = [&](TileRegs& R, int t0) {
    if constexpr (KVB) load_tile_bf16(R, a, b, h, t0, tid, t_end);
    else load_tile(R, a, bh, t0, tid, t_end);
  };
  const auto put = [&](const TileRegs& R, int bf) {
    if constexpr (KVB) store_tile_bf16<BF16>(R, Kl[bf], Vl[bf], KS[bf], VS[bf], tid, a.q_mul);
    else store_tile<BF16>(R, Kl[bf], Vl[bf], KS[bf], VS[bf], tid, a.q_mul);
  };
  // unconditional even for an empty range (lo >= t_end): every load then fails
  // its liveness test and reads nothing; a branch here costs the int8 kernel
  // 88 bytes of register spills
  TileRegs R;
  fetch(R, lo);
  put(R, 0);
  __syncthreads();

  // Software pipeline over 32-token units (four per 128-token tile): the
  // scores of unit k+1 are computed on the matrix cores while the VALU runs
  // the softmax of unit k, so every unit's Q·Kᵀ overlaps another unit's
  // softmax.  A tile's last unit is finished (softmax + P·V) in the next
  // iteration, from the tile's buffer, which is refilled only after a barrier.
  v4f sc[2][2][2];    // scores of two units in flight: [unit parity][rt][j]
  bool pend = false;  // the previous unit awaits its softmax + P·V
  int pend_t = 0;
  int buf = 0;
  const int qabs0 = P + q0;
  // a unit needs the mask loop if it reaches a query block's diagonal, the
  // cache end, or (sliding window) lies before some query's window start
  const auto needs_mask = [&](int tu) {
    return tu + 32 > qabs0 || tu + 32 > t_end || (window > 0 && tu < qabs0 + PF_QB - window);
  };
  for (int t0 = lo; t0 < t_end; t0 += PF_KT) {
    const bool more = t0 + PF_KT < t_end;
    if (more) fetch(R, t0 + PF_KT);  // in flight during this tile
    if (active) {
#pragma unroll
      for (int u = 0; u < PF_KT / 32; ++u) {
        const int tu = t0 + 32 * u;
        const bool live = tu < t_end;
        if (live) qk_unit<BF16>(Kl[buf] + 32 * u * PF_KROW, qop, sc[u & 1], c, g);
        if (pend) {
          // the unit before: this tile's unit u - 1, or the previous tile's last
          const int pb_ = u == 0 ? buf ^ 1 : buf, po = u == 0 ? PF_KT - 32 : 32 * (u - 1);
          softmax_pv_unit<VROW, EXACT>(sc[(u + 1) & 1], Vl[pb_] + po, KS[pb_] + po, VS[pb_] + po, m_use, thr, l_run,
                                acc, pend_t, t_end, qabs0, a.causal, window, needs_mask(pend_t), c, g);
        }
        pend = live;
        pend_t = tu;
      }
    }
    if (more) {
      // Other waves may still be finishing the previous tile's last unit,
      // which reads the other buffer: all of them pass this barrier before it
      // is refilled.
      __syncthreads();
      put(R, buf ^ 1);
      __syncthreads();
      buf ^= 1;
    }
  }
  // still pending: the last tile's last unit (every unit of a tile is visited,
  // and a tile has an even number of units, so its scores are in sc[1])
  if (active && pend)
    softmax_pv_unit<VROW, EXACT>(sc[1], Vl[buf] + PF_KT - 32, KS[buf] + PF_KT - 32, VS[buf] + PF_KT - 32, m_use, thr,
                          l_run, acc, pend_t, t_end, qabs0, a.causal, window, needs_mask(pend_t), c, g);

  if (!active) return;
  if (a.S > 1) {
    // ---------------- unnormalised partial of this split ----------------
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const float l = sum_xor32(sum_xor16(l_run[rt]));
      const float M = thr[rt] == NEG_INF ? NEG_INF : m_use[rt];  // -inf: no visible key in this split
      const int qr = q0 + 16 * rt + c;
      if (qr < a.L) {
        const int64_t row = ((((int64_t)bh * a.S + split) * a.nqb + qb) * 8 + w) * PF_QB + 16 * rt + c;
        float* o = a.ws_acc + row * HEAD_DIM + 4 * g;
#pragma unroll
        for (int n = 0; n < 8; ++n) *(v4f*)(o + 16 * n) = acc[n][rt];
        if (g == 0) *(v2f*)(a.ws_stat + row * 2) = (v2f){M, l};
      }
    }
    return;
  }
  // ---------------- normalise and write ----------------
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    float l = l_run[rt];
    l = sum_xor32(sum_xor16(l));
    float M = thr[rt] == NEG_INF ? NEG_INF : m_use[rt];  // -inf: no visible key
    if (a.sinks != nullptr) {
      const float sink = a.sinks[hq] * LOG2E;
      const float Mn = fmaxf(M, sink);
      const float f = M == NEG_INF ? 0.f : __builtin_amdgcn_exp2f(M - Mn);
      l = l * f + __builtin_amdgcn_exp2f(sink - Mn);
#pragma unroll
      for (int n = 0; n < 8; ++n) acc[n][rt] *= f;
    }
    const float inv = l > 0.f ? 1.f / l : 1.f;
    const int qr = q0 + 16 * rt + c;
    if (qr < a.L) {
      float* o = a.out + (((int64_t)b * a.Hq + hq) * a.L + qr) * HEAD_DIM + 4 * g;
#pragma unroll
      for (int n = 0; n < 8; ++n) *(v4f*)(o + 16 * n) = acc[n][rt] * inv;
    }
  }
}

// Merge of the key splits (S > 1): one wavefront per (query, query head,
// batch); lane k owns the statistics of split k, the weights go through LDS,
// and lane l sums dims 2l, 2l + 1 over the splits.  The sink logit joins here.
__global__ __launch_bounds__(64) void prefill_merge_kernel(const PrefillArgs a) {
  __shared__ float wts[PREFILL_MAX_SPLITS];
  const int i = blockIdx.x, hq = blockIdx.y, b = blockIdx.z, lane = threadIdx.x;
  const int h = hq / a.G, w = hq % a.G, qb = i / PF_QB, r = i % PF_QB;
  const int64_t bh = (int64_t)b * a.Hkv + h;
  const auto row = [&](int sp) { return ((((bh * a.S + sp) * a.nqb + qb) * 8 + w) * PF_QB) + r; };
  float m = NEG_INF, l = 0.f;
  if (lane < a.S) {
    const v2f st = *(const v2f*)(a.ws_stat + row(lane) * 2);
    m = st[0];
    l = st[1];
  }
  const float sink = a.sinks != nullptr ? a.sinks[hq] * LOG2E : NEG_INF;
  const float M = fmaxf(wave_max(m), sink);
  const float f = (m == NEG_INF || M == NEG_INF) ? 0.f : __builtin_amdgcn_exp2f(m - M);
  float z = wave_sum(f * l);
  if (sink != NEG_INF) z += __builtin_amdgcn_exp2f(sink - M);
  wts[lane] = f;  // 0 for lanes past the last split
  __syncthreads();
  // 16 independent loads in flight per round (slots past the last split read
  // its row again and weigh it 0), not one memory round trip per split
  v2f acc = {0.f, 0.f};
  for (int s0 = 0; s0 < a.S; s0 += 16) {
    v2f x[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) x[k] = *(const v2f*)(a.ws_acc + row(min(s0 + k, a.S - 1)) * HEAD_DIM + 2 * lane);
#pragma unroll
    for (int k = 0; k < 16; ++k) acc += wts[min(s0 + k, PREFILL_MAX_SPLITS - 1)] * x[k];
  }
  const float inv = z > 0.f ? 1.f / z : 1.f;
  *(v2f*)(a.out + (((int64_t)b * a.Hq + hq) * a.L + i) * HEAD_DIM + 2 * lane) = acc * inv;
}

PrefillPlan prefill_plan(const PrefillArgs& a, int requested) {
  PrefillPlan p{};
  p.nqb = (a.L + PF_QB - 1) / PF_QB;
  const int kt = a.kv_bf16 ? PfTile<true>::KT : PfTile<false>::KT;
  // keys any query block scans: from the first block's window start to T
  const int64_t P = a.T - a.L;
  const int64_t lo = (a.kv_bf16 && a.window > 0) ? std::max<int64_t>(0, P - a.window + 1) / kt * kt : 0;
  const int64_t tiles = (a.T - lo + kt - 1) / kt;
  int S = requested;
  if (S <= 0) {
    // one workgroup per CU: split only a grid below half the chip, and keep
    // at least two tiles per split
    const int64_t nwg = (int64_t)p.nqb * a.Hkv * a.B;
    S = nwg >= 128 ? 1 : (int)std::min<int64_t>(PREFILL_MAX_SPLITS, (256 + nwg - 1) / nwg);
    S = (int)std::min<int64_t>(S, std::max<int64_t>(1, tiles / 2));
  }
  S = std::max(1, std::min(S, PREFILL_MAX_SPLITS));
  S = (int)std::min<int64_t>(S, std::max<int64_t>(1, tiles));
  const int64_t per = (tiles + S - 1) / S;  // tiles per split
  p.S = (int)((tiles + per - 1) / per);
  p.split_lo = lo;
  p.split_len = per * kt;
  if (p.S == 1) {  // one range covering everything
    p.split_lo = 0;
    p.split_len = a.T + kt;
  }
  return p;
}

size_t prefill_ws_bytes(int B, int Hkv, int nqb, int S) {
  if (S <= 1) return 0;
  const size_t rows = (size_t)B * Hkv * S * nqb * 8 * PF_QB;
  return rows * HEAD_DIM * 4 + rows * 2 * 4;
}

template <bool EXACT>
static void launch_prefill_pv(const PrefillArgs& a, dim3 grid, dim3 block, hipStream_t stream) {
  if (a.kv_bf16) {
    if (a.q_dtype == DT_BF16) hipLaunchKernelGGL((prefill_kernel<true, true, EXACT>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((prefill_kernel<false, true, EXACT>), grid, block, 0, stream, a);
  } else {
    if (a.q_dtype == DT_BF16) hipLaunchKernelGGL((prefill_kernel<true, false, EXACT>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((prefill_kernel<false, false, EXACT>), grid, block, 0, stream, a);
  }
}

// Fewest keys any query row of the launch sees: the first row's causal
// prefix (and at most the window), or all T keys without a causal mask.
static int64_t fewest_visible_keys(const PrefillArgs& a) {
  int64_t n = a.causal ? a.T - a.L + 1 : a.T;
  if (a.kv_bf16 && a.window > 0 && a.window < n) n = a.window;
  return n;
}

hipError_t launch_prefill(const PrefillArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)(a.nqb * a.S), a.Hkv, a.B), block(512);
  if (fewest_visible_keys(a) < EXACT_PV_BELOW) launch_prefill_pv<true>(a, grid, block, stream);
  else launch_prefill_pv<false>(a, grid, block, stream);
  if (a.S > 1) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(prefill_merge_kernel, dim3((unsigned)a.L, a.Hq, a.B), dim3(64), 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace rec
