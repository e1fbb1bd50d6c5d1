// Chunked prefill attention over the quantized or bf16 KV cache on bf16 /
// fp16 matrix cores (gfx950).
//
// Restates the prefill branch of Attention.__call__
// (engine/src/rec_mlx/model.py:191-203): the new tokens were quantize-appended
// first (model.py:177-178), then the L new queries attend over the whole
// cache, the new tokens included, with the causal "string" mask of
// model.py:122-125 (query i sits at position T-L+i) and the per-head sink
// logit in the softmax denominator.  The reference dequantizes the cache to
// the query dtype (model.py:194-195) and runs one SDPA; here every K/V tile is
// dequantized into LDS on the way from HBM, never written back:
//   * int8 K/V: the codes enter the matrix products exactly (|q| <= 127) and
//     the row scales are applied outside them, the K scale to the scores, the
//     V scale folded into the probabilities before their rounding;
//   * 4-bit and affine K/V: x̂ = (q - z)·s or q·s + b in float32, rounded to
//     the query dtype as the reference's dequantization does (V then held
//     as fp16 for the P·V product);
//   * a bf16 cache (KVStorage views, ring windows): the values as they are.
// Q·K^T runs on bf16 MFMAs for bf16 queries (fp16 for fp16 queries); P·V on
// fp16 MFMAs, whose 11-bit significand keeps each rounded P' within 2^-12
// (and a second MFMA carries the rounding remainder for rows that see few
// keys, EXACT_PV_BELOW).
//
// Work decomposition.  Grid (ceil(L*G/256) x key splits, Hkv, B), 512
// threads = 8 wavefronts.  The rows of a KV head's attention are its (query,
// head) pairs, query-major (row query*G + head over the G query heads of the
// GQA group); a workgroup takes 256 consecutive rows as 16 row tiles of 16,
// and wave w owns tiles w and w + 8.  A chunk of a few queries thus fills
// its row tiles with those queries' heads instead of padding every head to a
// tile, and a wave whose tiles lie past the last row skips them.
//
// K/V tiles of 128 tokens (64 for a bf16 cache) are dequantized into
// double-buffered LDS and shared by the 8 waves, which compute a tile in
// 32-token units, software-pipelined (one unit's Q·K^T on the matrix cores
// while the previous unit's softmax runs on the VALU); each burst issues its
// LDS operand reads together ahead of its MFMAs, so it waits for the LDS
// once.  Each tile's raw bytes are fetched a whole tile ahead and dequantized
// into the other buffer between two barriers at the end of the current tile;
// its scale bytes reach the converting threads through a small LDS staging
// area.  (Spreading the conversion over the units, behind their Q·K^T MFMAs,
// was measured no faster: with two waves per SIMD the kernel is bound by each
// wave's in-order chain of LDS reads, MFMAs and softmax, not by the
// conversion's VALU work.)  A grid too small to fill the chip (a short chunk
// over a long cache) splits the keys: each workgroup writes an unnormalised
// partial and prefill_merge_kernel combines the splits as the decode's merge
// does (megakernel.py:276-318).
//
// S^T = K Q^T on 16x16x32 MFMAs (A = 16 tokens x 32 dims from LDS, B = Q^T held
// in registers), which leaves lane (c, g) with the scores of query row c for
// tokens 16j + 4g + i -- the order the cache keeps V in inside a 32-token
// block.  P·V then takes A = V^T straight from LDS (dims x tokens, cache
// order) and B = P'^T from the lane's own registers.
#include <algorithm>
#include <type_traits>

#include "kernels.h"

namespace rec {

constexpr int PF_ROWS = PREFILL_BLOCK_ROWS;  // (query, head) rows per workgroup: 16 tiles of 16
constexpr int PF_KROW = 144;  // LDS row pitch of K (elements): 128 + 16 pad

// Tile geometry per cache format pair.
template <int KF, int VF>
struct PfGeom {
  static constexpr bool BF = KF == FMT_BF;
  static constexpr int KT = BF ? 64 : 128;  // tokens per tile (a bf16 tile moves twice the bytes per token)
  static constexpr int U = KT / 32;         // 32-token units per tile
  static constexpr int VROW = KT + 16;      // LDS row pitch of V (positions + 16 pad)
  // A bf16 cache holds V token-major: its tile keeps V as rows (token at
  // block position within its 32-token unit, 144-element pitch) and P·V reads
  // the Vᵀ operand with transposing LDS reads; the quantized layouts already
  // group a dim's tokens, so their tiles hold V as [dim][position] rows.
  static constexpr bool VTR = BF;
  static constexpr int VPB = 144;
  static constexpr int K_ELEMS = KT * PF_KROW;
  static constexpr int V_ELEMS = VTR ? KT * VPB : HEAD_DIM * VROW;
  // element offset of unit u's V in the tile
  static constexpr int vunit(int u) { return VTR ? 32 * u * VPB : 32 * u; }
  // V^T operands of a unit read ahead of its softmax (of 8): all of them,
  // or half where the registers would spill in the hot loop (a mixed
  // int8/uint4 pair; the affine pair with the exact P·V); the bf16 cache's
  // transposed reads measured fastest issued at the P·V
  static constexpr int vpre(bool exact) {
    return VTR ? 0 : ((KF == 8 && VF == 4) || (KF == 4 && VF == 8) || (exact && is_a8(KF))) ? 4 : 8;
  }
  // Scale bytes per 32-token block, per staged region: [K scales][K zeros][V scales][V zeros]
  // (int8: one fp16 per token; uint4: [4 groups][32 slots] fp16 scales, zero-points alike;
  // affine: [scale, bias][2 groups][32 slots] bf16 in the scales region).
  static constexpr int KS_B = KF == 8 ? 64 : (KF == 4 || is_a8(KF)) ? 256 : 0;
  static constexpr int KZ_B = KF == 4 ? 256 : 0;
  static constexpr int VS_B = VF == 8 ? 64 : (VF == 4 || is_a4(VF)) ? 256 : 0;
  static constexpr int VZ_B = VF == 4 ? 256 : 0;
  static constexpr int OFF_KZ = 4 * KS_B, OFF_VS = OFF_KZ + 4 * KZ_B, OFF_VZ = OFF_VS + 4 * VS_B;
  static constexpr int STAGE = OFF_VZ + 4 * VZ_B;  // <= 4096
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
  static __device__ __forceinline__ elem from_float(float x) { return (__bf16)x; }  // round to nearest even
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

// fp16 value of a dequantized V element as the reference holds it: rounded
// to the query dtype first (bf16 queries), then widened to the fp16 P·V
// operand (exact inside fp16's range).
template <bool BF16>
__device__ __forceinline__ _Float16 v_elem(float x) {
  if constexpr (BF16) return (_Float16)(float)(__bf16)x;
  else return (_Float16)x;
}

// One thread's share of a tile's raw bytes, as loaded from HBM.
struct TileRegs {
  v4i k[2];  // int8 / affine-8 K: two 16-byte runs; uint4 K: k[0] = two 8-byte runs; bf16: two 16-byte rows
  v4i v[2];  // int8 V: two 16-byte runs; 4-bit V: v[0] = two 8-byte runs; bf16: two 16-byte rows
  v2i sc;    // 8 bytes of the tile's staged scale regions
};

// ---------------------------------------------------------------- loads --
// Thread -> bytes, per format (tile of KT tokens at t0, a multiple of KT):
//   int8 / affine-8 K, int8 V: byte o = 16 (tid % 256) of blocks 2p + tid / 256, p = 0, 1;
//   uint4 K: token t = tid / 4, dims 32 (tid % 4) .. +31 (runs 2(q&1), +1 of half q/2);
//   4-bit V: block tid / 128, dims 16(4N + 2kk + k) + c (k = 0, 1), positions 8g .. 8g+7
//     for g = 2gg, 2gg+1 (N = bit 6, c = bits 2-5, kk = bit 1, gg = bit 0 of tid);
//   bf16: 16-byte chunks tid and tid + 512 of the 64-token tile, chunk = (token, 8 dims);
//   scales: 8 bytes at staged offset 8 tid (regions contiguous per (b, h) in HBM).
template <int KF, int VF>
__device__ __forceinline__ void load_tile(TileRegs& R, const PrefillArgs& a, int b, int h, int64_t bh, int t0,
                                          int tid, int t_end) {
  typedef PfGeom<KF, VF> GEO;
  const int64_t blk0 = bh * (a.cap / BLOCK_T) + (t0 >> 5);  // first cache block of the tile
  if constexpr (KF == FMT_BF) {
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
    return;
  } else {
    if constexpr (KF == 8 || is_a8(KF)) {
      const int o = (tid & 255) * 16;
#pragma unroll
      for (int part = 0; part < 2; ++part) {
        const int bk = 2 * part + (tid >> 8);
        const bool live = t0 + 32 * bk < t_end;
        const int8_t* kb = (const int8_t*)a.kq + (blk0 + bk) * 4096;
        R.k[part] = live ? __builtin_nontemporal_load((const v4i*)(kb + o)) : (v4i){0, 0, 0, 0};
      }
    } else {  // uint4 K
      const int t = tid >> 2, q = tid & 3, bk = t >> 5;
      const bool live = t0 + 32 * bk < t_end;
      const uint8_t* kb = (const uint8_t*)a.kq + (blk0 + bk) * 2048 + (t & 31) * 64 + (2 * (q & 1)) * 16 + (q >> 1) * 8;
      const v2i lo = live ? __builtin_nontemporal_load((const v2i*)kb) : (v2i){0, 0};
      const v2i hi = live ? __builtin_nontemporal_load((const v2i*)(kb + 16)) : (v2i){0, 0};
      R.k[0] = (v4i){lo[0], lo[1], hi[0], hi[1]};
    }
    if constexpr (VF == 8) {
      const int o = (tid & 255) * 16;
#pragma unroll
      for (int part = 0; part < 2; ++part) {
        const int bk = 2 * part + (tid >> 8);
        const bool live = t0 + 32 * bk < t_end;
        const int8_t* vb = (const int8_t*)a.vq + (blk0 + bk) * 4096;
        R.v[part] = live ? __builtin_nontemporal_load((const v4i*)(vb + o)) : (v4i){0, 0, 0, 0};
      }
    } else {  // 4-bit V (uint4 or affine)
      const int bk = tid >> 7, N = (tid >> 6) & 1, c = (tid >> 2) & 15, kk = (tid >> 1) & 1, gg = tid & 1;
      const bool live = t0 + 32 * bk < t_end;
      const uint8_t* vb = (const uint8_t*)a.vq + (blk0 + bk) * 2048 + N * 1024 + (c * 4 + 2 * gg) * 16 + kk * 8;
      const v2i g0 = live ? __builtin_nontemporal_load((const v2i*)vb) : (v2i){0, 0};
      const v2i g1 = live ? __builtin_nontemporal_load((const v2i*)(vb + 16)) : (v2i){0, 0};
      R.v[0] = (v4i){g0[0], g0[1], g1[0], g1[1]};
    }
    // scale bytes: region (K scales, K zeros, V scales, V zeros) of the staged tile
    R.sc = (v2i){0, 0};
    const int off = 8 * tid;
    if (off < GEO::STAGE) {
      // the region's base chosen by selects (a branch chain on this lane-varying
      // offset became a private array of the four pointers, in scratch memory)
      const bool r1 = off >= GEO::OFF_KZ, r2 = off >= GEO::OFF_VS, r3 = off >= GEO::OFF_VZ;
      const uint64_t base = r3 ? (uint64_t)a.vz : r2 ? (uint64_t)a.vs : r1 ? (uint64_t)a.kz : (uint64_t)a.ks;
      const int start = r3 ? GEO::OFF_VZ : r2 ? GEO::OFF_VS : r1 ? GEO::OFF_KZ : 0;
      const int per = r3 ? GEO::VZ_B : r2 ? GEO::VS_B : r1 ? GEO::KZ_B : GEO::KS_B;
      const int rel = off - start;
      const int bk = rel / per;
      // a global-memory pointer: through a generic one this would be a flat
      // load, which the LDS waits of the whole next tile would count too
      typedef const __attribute__((address_space(1))) v2i global_v2i;
      if (t0 + 32 * bk < t_end) R.sc = *(global_v2i*)(base + (uint64_t)(blk0 * per + rel));
    }
  }
}

// -------------------------------------------------------------- convert --
// The thread's raw bytes -> dequantized LDS tile (buffer of tile tokens KT).
// Phase 0: K rows [token][dim]; phase 1: V [dim][cache position]; phase 2:
// the K / V scale arrays of the softmax (int8: the row scales, the K one
// times the softmax scale; dequantized formats: the softmax scale and 1).
template <bool BF16, int KF, int VF, int PHASE>
__device__ __forceinline__ void convert_tile(const TileRegs& R, typename MT<BF16>::elem* Kl, _Float16* Vl, float* KS,
                                             float* VS, const char* stage, int tid, float q_mul) {
  typedef PfGeom<KF, VF> GEO;
  typedef typename MT<BF16>::elem E;
  constexpr int VROW = GEO::VROW;
  if constexpr (KF == FMT_BF) {
    if constexpr (PHASE == 0) {
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
      }
    } else if constexpr (PHASE == 1) {
      // V rows as fp16 (the P·V operand type), token t of the tile at row
      // 32 (t / 32) + block_pos(t % 32)
#pragma unroll
      for (int part = 0; part < 2; ++part) {
        const int id = part * 512 + tid, tok = id >> 4, d0 = (id & 15) * 8;
        const int row = (tok & ~31) + block_pos(tok & 31);
        v8h vh;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t w = (uint32_t)R.v[part][e];
          vh[2 * e] = (_Float16)__builtin_bit_cast(float, w << 16);
          vh[2 * e + 1] = (_Float16)__builtin_bit_cast(float, w & 0xffff0000u);
        }
        *(v8h*)(Vl + row * GEO::VPB + d0) = vh;
      }
    } else {
      if (tid < 2 * GEO::KT) (tid < GEO::KT ? KS : VS)[tid & (GEO::KT - 1)] = tid < GEO::KT ? q_mul : 1.f;
    }
    return;
  } else {
    if constexpr (PHASE == 0) {
      if constexpr (KF == 8 || is_a8(KF)) {
        // block run o = [half m][token r][64 bytes]: dims 64m + e0 .. +15 of token r
        const int o = (tid & 255) * 16, m = o >> 11, r = (o & 2047) >> 6, e0 = o & 63;
#pragma unroll
        for (int part = 0; part < 2; ++part) {
          const int bk = 2 * part + (tid >> 8);
          E* dst = Kl + (32 * bk + r) * PF_KROW + 64 * m + e0;
          if constexpr (KF == 8) {
            if constexpr (BF16) {
#pragma unroll
              for (int w = 0; w < 4; ++w)
#pragma unroll
                for (int bb = 0; bb < 4; ++bb)
                  dst[4 * w + bb] = (__bf16)(float)(int8_t)((uint32_t)R.k[part][w] >> (8 * bb));
            } else {  // fp16: the codes glued under the exponent of 1024 (exact)
              *(v8h*)dst = i8x8_to_h8((uint32_t)R.k[part][0], (uint32_t)R.k[part][1]);
              *(v8h*)(dst + 8) = i8x8_to_h8((uint32_t)R.k[part][2], (uint32_t)R.k[part][3]);
            }
          } else {  // affine 8-bit: x = q·s + b, (s, b) of group m at the token's slot
            const int slot = s4_slot(block_pos(r));
            const uint16_t* sb = (const uint16_t*)(stage + bk * 256);
            const float sc = meta_bits<meta_f16(KF)>(sb[m * 32 + slot]);
            const float bi = meta_bits<meta_f16(KF)>(sb[64 + m * 32 + slot]);
            // (v_cvt_f32_ubyte reads each code byte directly: one conversion
            // and one fma per element; the fp16 unpack measured 3% slower here)
#pragma unroll
            for (int w = 0; w < 4; ++w)
#pragma unroll
              for (int bb = 0; bb < 4; ++bb)
                dst[4 * w + bb] = MT<BF16>::from_float(__builtin_fmaf(
                    (float)(((uint32_t)R.k[part][w] >> (8 * bb)) & 0xffu), sc, bi));
          }
        }
      } else {  // uint4 K: token t, group q (dims 32q .. 32q+31); x = (q - z)·s
        const int t = tid >> 2, q = tid & 3, bk = t >> 5, slot = s4_slot(block_pos(t & 31));
        const uint16_t* ss = (const uint16_t*)(stage + bk * 256);
        const uint16_t* zz = (const uint16_t*)(stage + GEO::OFF_KZ + bk * 256);
        const float sc = half_bits_to_float(ss[q * 32 + slot]);
        const _Float16 zh = __builtin_bit_cast(_Float16, zz[q * 32 + slot]);
        const v2h zl = {(_Float16)1024.0f + zh, (_Float16)1024.0f + zh};
        const v2h zu = {(_Float16)64.0f + zh, (_Float16)64.0f + zh};
        E* dst = Kl + t * PF_KROW + 32 * q;
        // word w: dims 8w .. 8w+7 of the group, byte i holding dims 8w + 2i (low
        // nibble) and 8w + 2i + 1.  The decode's fp16 unpack: a low nibble under
        // the exponent of 1024, a high one under that of 64, minus that offset
        // and z, is q - z exactly, for the dim pairs (i, i+4); x̂ = (q - z)·s
        // exactly in fp32 from the fp16 operand (v_fma_mix), rounded once to the
        // query type
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t W = (uint32_t)R.k[0][w], W8 = W >> 8;
          const v2h d04 = __builtin_bit_cast(v2h, and_or(W, 0x000f000fu, 0x64006400u)) - zl;
          const v2h d15 = __builtin_bit_cast(v2h, and_or(W, 0x00f000f0u, 0x54005400u)) - zu;
          const v2h d26 = __builtin_bit_cast(v2h, and_or(W8, 0x000f000fu, 0x64006400u)) - zl;
          const v2h d37 = __builtin_bit_cast(v2h, and_or(W8, 0x00f000f0u, 0x54005400u)) - zu;
          E* o = dst + 8 * w;
          o[0] = MT<BF16>::from_float(__builtin_fmaf((float)d04[0], sc, 0.f));
          o[1] = MT<BF16>::from_float(__builtin_fmaf((float)d15[0], sc, 0.f));
          o[2] = MT<BF16>::from_float(__builtin_fmaf((float)d26[0], sc, 0.f));
          o[3] = MT<BF16>::from_float(__builtin_fmaf((float)d37[0], sc, 0.f));
          o[4] = MT<BF16>::from_float(__builtin_fmaf((float)d04[1], sc, 0.f));
          o[5] = MT<BF16>::from_float(__builtin_fmaf((float)d15[1], sc, 0.f));
          o[6] = MT<BF16>::from_float(__builtin_fmaf((float)d26[1], sc, 0.f));
          o[7] = MT<BF16>::from_float(__builtin_fmaf((float)d37[1], sc, 0.f));
        }
      }
    } else if constexpr (PHASE == 1) {
      if constexpr (VF == 8) {
        // run o = [n/2][c][position group pg][n%2][8 positions]: positions
        // 8pg .. 8pg+7 of dims 16n + c, n = n0 and n0 + 1
        const int o = (tid & 255) * 16, n0 = 2 * (o >> 10), cc = (o >> 6) & 15, pg = (o >> 4) & 3;
#pragma unroll
        for (int part = 0; part < 2; ++part) {
          const int bk = 2 * part + (tid >> 8);
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            _Float16* dst = Vl + (16 * (n0 + half) + cc) * VROW + 32 * bk + 8 * pg;
            *(v8h*)dst = i8x8_to_h8((uint32_t)R.v[part][2 * half], (uint32_t)R.v[part][2 * half + 1]);
          }
        }
      } else {  // 4-bit V: dims 16(4N + 2kk + k) + c, positions 8g + e of block bk
        const int bk = tid >> 7, N = (tid >> 6) & 1, c = (tid >> 2) & 15, kk = (tid >> 1) & 1, gg = tid & 1;
        const int grp = VF == 4 ? 2 * N + kk : N;  // the dims' scale group (32 or 64 dims)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int g = 2 * gg + j;
          // slots 8g .. 8g+7 hold positions 8g + {0, 4, 1, 5, 2, 6, 3, 7}
          // (s4_slot): dword e of a run is the (scale, zero / bias) pair of
          // positions (e, e+4), the pair the fp16 unpack yields at step e
          const v4i s4 = *(const v4i*)(stage + GEO::OFF_VS + bk * 256 + (grp * 32 + 8 * g) * 2);
          const v4i z4 = VF == 4 ? *(const v4i*)(stage + GEO::OFF_VZ + bk * 256 + (grp * 32 + 8 * g) * 2)
                                 : *(const v4i*)(stage + GEO::OFF_VS + bk * 256 + (64 + grp * 32 + 8 * g) * 2);
          const v2h k1024 = {(_Float16)1024.0f, (_Float16)1024.0f}, k64 = {(_Float16)64.0f, (_Float16)64.0f};
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            const uint32_t W = (uint32_t)R.v[0][2 * j + k], W8 = W >> 8;  // position 8g + e at nibble e
            v8h out;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              // copies first: a bit_cast of a vector subscript reads element 0
              const uint32_t sw = (uint32_t)s4[e], zw = (uint32_t)z4[e];
              const uint32_t t = (e & 1) ? and_or(e < 2 ? W : W8, 0x00f000f0u, 0x54005400u)
                                         : and_or(e < 2 ? W : W8, 0x000f000fu, 0x64006400u);
              float x0, x1;
              if constexpr (VF == 4) {  // (q - z)·s, exact in fp32 from the fp16 q - z
                const v2h d = __builtin_bit_cast(v2h, t) - (__builtin_bit_cast(v2h, zw) + ((e & 1) ? k64 : k1024));
                const v2h sv = __builtin_bit_cast(v2h, sw);
                x0 = __builtin_fmaf((float)d[0], (float)sv[0], 0.f);
                x1 = __builtin_fmaf((float)d[1], (float)sv[1], 0.f);
              } else {  // q·s + b in one fma
                const v2h qv = __builtin_bit_cast(v2h, t) - ((e & 1) ? k64 : k1024);
                constexpr bool F16 = meta_f16(VF);
                x0 = __builtin_fmaf((float)qv[0], meta_lo<F16>(sw), meta_lo<F16>(zw));
                x1 = __builtin_fmaf((float)qv[1], meta_hi<F16>(sw), meta_hi<F16>(zw));
              }
              out[e] = v_elem<BF16>(x0);
              out[e + 4] = v_elem<BF16>(x1);
            }
            *(v8h*)(Vl + (16 * (4 * N + 2 * kk + k) + c) * VROW + 32 * bk + 8 * g) = out;
          }
        }
      }
    } else {
      if (tid < 2 * GEO::KT) {
        const bool is_k = tid < GEO::KT;
        const int t = tid & (GEO::KT - 1);
        float x = is_k ? q_mul : 1.f;
        if ((is_k && KF == 8) || (!is_k && VF == 8)) {
          const uint16_t* s8 = (const uint16_t*)(stage + (is_k ? 0 : GEO::OFF_VS));
          x *= half_bits_to_float(s8[(t >> 5) * 32 + block_pos(t & 31)]);
        }
        (is_k ? KS : VS)[t] = x;
      }
    }
  }
}

// S^T = K Q^T for one 32-token unit of one wave: its first NRT row tiles of
// 16; lane (c, g) receives the scores of row c of each tile for tokens
// 16j + 4g + i of the unit.
template <bool BF16, int NRT>
__device__ __forceinline__ void qk_unit(const typename MT<BF16>::elem* K, const typename MT<BF16>::vec (&qop)[2][4],
                                        v4f (&s4)[2][2], int c, int g) {
  typedef typename MT<BF16>::vec V8;
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
    for (int j = 0; j < 2; ++j) s4[rt][j] = (v4f){0.f, 0.f, 0.f, 0.f};
  // all eight operand reads first, so that the MFMAs wait for the LDS once
  V8 ka[4][2];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int j = 0; j < 2; ++j) ka[ks][j] = *(const V8*)(K + (16 * j + c) * PF_KROW + 32 * ks + 8 * g);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt) s4[rt][j] = MT<BF16>::mfma(ka[ks][j], qop[rt][ks], s4[rt][j]);
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
template <int VROW, bool VTR, bool EXACT, int NRT, int VPRE, bool BIAS>
__device__ __forceinline__ void softmax_pv_unit(const v4f (&s4)[2][2], const _Float16* Vv, const float* KS,
                                                const float* VS, float (&m_use)[2], float (&thr)[2],
                                                float (&l_run)[2], v4f (&acc)[8][2], int t0, int t_end,
                                                const int (&qabs)[2], int causal, int window, bool mask,
                                                int c, int g, __amdgpu_buffer_rsrc_t rb, const uint32_t (&brow)[2]) {
  v8h pb[2], pl[2];  // P'^T: high parts, and (EXACT) the remainders
  // BIAS: the rows' bias (a mask array, natural-log units) for the lane's
  // tokens t0 + 16j + 4g + i, from HBM first of all
  v4f bz[2][2];
  if constexpr (BIAS) {
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bz[rt][j] = __builtin_bit_cast(v4f, ld128<0>(rb, (brow[rt] + (uint32_t)(t0 + 16 * j + 4 * g)) * 4u, 0));
  }
  // The unit's LDS reads first: the row scales and the first VPRE of the
  // eight V^T operands, whose latency the softmax arithmetic then covers
  // (one wait instead of one per pair of operands).
  v4f ksc[2], vsc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    ksc[j] = *(const v4f*)(&KS[16 * j + 4 * g]);
    vsc[j] = *(const v4f*)(&VS[16 * j + 4 * g]);
  }
  v8h va[8];
  const int sk = c >> 2, sa = c & 3;  // transposed reads: rows 8g + sk (+4), dims 16n + 4sa
  const auto load_va = [&](int n) {
    if constexpr (VTR) {
      // in a group of 16 lanes, lane 4a+b receives element b of the 8-byte
      // rows addressed by lanes 4k+a: lane c gets dim 16n + c of rows 8g .. 8g+7
      typedef __fp16 v4fp16 __attribute__((__vector_size__(4 * sizeof(__fp16))));
      typedef __attribute__((address_space(3))) v4fp16 lds_v4fp16;
      const _Float16* base = Vv + (8 * g + sk) * 144 + 16 * n + 4 * sa;
      const v2i r0 = __builtin_bit_cast(v2i, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_v4fp16*)base));
      const v2i r1 = __builtin_bit_cast(v2i, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_v4fp16*)(base + 4 * 144)));
      va[n] = __builtin_bit_cast(v8h, (v4i){r0[0], r0[1], r1[0], r1[1]});
    } else {
      va[n] = *(const v8h*)(Vv + (16 * n + c) * VROW + 8 * g);
    }
  };
#pragma unroll
  for (int n = 0; n < VPRE; ++n) load_va(n);
  if constexpr (VPRE > 0) __builtin_amdgcn_sched_barrier(0);
  // Range: P' = p·s feeds an fp16 operand, finite while p·s < 65504.  A V
  // scale of 2 or more among the lane's tokens (fp32 exponent bit 30;
  // |v| >= 254) makes its bound 0 for this unit, so its p <= 1 and
  // P' <= s <= 65504.
  bool big;
  {
    const v4i o = __builtin_bit_cast(v4i, vsc[0]) | __builtin_bit_cast(v4i, vsc[1]);
    big = ((uint32_t)(o[0] | o[1] | o[2] | o[3]) & 0x40000000u) != 0;
  }
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt) {
    // scale (K scale x softmax scale) and offset in one fma, mask, online
    // softmax per row (lane column c of tile rt; its query sits at qabs[rt])
    float t[8];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) t[4 * j + i] = __builtin_fmaf(s4[rt][j][i], ksc[j][i], -m_use[rt]);
    if constexpr (BIAS) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) t[4 * j + i] = __builtin_fmaf(bz[rt][j][i], LOG2E, t[4 * j + i]);
    }
    if (mask) {
      // first and last visible token of this row, relative to the lane's first token t0 + 4g
      const int last = (causal ? min(qabs[rt], t_end - 1) : t_end - 1) - t0 - 4 * g;
      const int first = window > 0 ? qabs[rt] - window + 1 - t0 - 4 * g : INT32_MIN;
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
    // B operand of P·V: k index 8g + 4j + i = cache position of token 16j + 4g + i
    float pr[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) pr[k] = __builtin_amdgcn_exp2f(t[k]);
    float lsum = pr[0];
#pragma unroll
    for (int k = 1; k < 8; ++k) lsum += pr[k];
    l_run[rt] += lsum;
    if constexpr (EXACT) {
      // P' = p·s rounded to fp16 once by v_fma_mix, straight into the
      // operand's halves (fewer registers than a multiply, a conversion and
      // a pack; the room goes to the V operands read ahead), then the
      // remainder
#pragma unroll
      for (int k = 0; k < 8; k += 2) {
        const int j = k >> 2, i = k & 3;
        uint32_t w;
        asm("v_fma_mixlo_f16 %0, %1, %2, 0" : "=v"(w) : "v"(pr[k]), "v"(vsc[j][i]));
        asm("v_fma_mixhi_f16 %0, %1, %2, 0" : "+v"(w) : "v"(pr[k + 1]), "v"(vsc[j][i + 1]));
        const v2h hh = __builtin_bit_cast(v2h, w);
        pb[rt][k] = hh[0];
        pb[rt][k + 1] = hh[1];
        pl[rt][k] = (_Float16)__builtin_fmaf(pr[k], vsc[j][i], -(float)hh[0]);
        pl[rt][k + 1] = (_Float16)__builtin_fmaf(pr[k + 1], vsc[j][i + 1], -(float)hh[1]);
      }
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) pb[rt][k] = (_Float16)(pr[k] * vsc[k >> 2][k & 3]);
    }
  }
  __builtin_amdgcn_s_setprio(1);  // as around the Q·Kᵀ burst
#pragma unroll
  for (int n = VPRE; n < 8; ++n) load_va(n);
#pragma unroll
  for (int n = 0; n < 8; ++n) {
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
      acc[n][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[n], pb[rt], acc[n][rt], 0, 0, 0);
      if constexpr (EXACT) acc[n][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[n], pl[rt], acc[n][rt], 0, 0, 0);
    }
  }
  __builtin_amdgcn_s_setprio(0);
}

// Q^T operands: lane column c of row tile rt holds the query row (qr[rt],
// head hq[rt]); k-step ks dims 32ks + 8g .. +7.
template <bool BF16>
__device__ __forceinline__ void load_query(typename MT<BF16>::vec (&qop)[2][4], const PrefillArgs& a, int b,
                                           const int (&hq)[2], const int (&qr)[2], int g) {
  typedef typename MT<BF16>::vec V8;
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int64_t base = (int64_t)b * a.q_sb + (int64_t)hq[rt] * a.q_sh + (int64_t)qr[rt] * a.q_st;
    const uint16_t* row = (const uint16_t*)a.q + base;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if (a.q_vec) {
        qop[rt][ks] = __builtin_bit_cast(V8, *(const v4i*)(row + 32 * ks + 8 * g));
      } else {
        v8s e;
#pragma unroll
        for (int i = 0; i < 8; ++i) e[i] = (short)row[32 * ks + 8 * g + i];
        qop[rt][ks] = __builtin_bit_cast(V8, e);
      }
    }
  }
}

// MM, the mask mode: 0 causal or none, 1 + a sliding window, 2 + a bias
// (mask array) read per unit and row
template <bool BF16, int KF, int VF, bool EXACT, int MM>
__global__ __launch_bounds__(512) void prefill_kernel(const PrefillArgs a) {
  typedef PfGeom<KF, VF> GEO;
  typedef typename MT<BF16>::elem E;
  typedef typename MT<BF16>::vec V8;
  constexpr int KT = GEO::KT, U = GEO::U, VROW = GEO::VROW;
  __shared__ __attribute__((aligned(16))) E Kl[2][GEO::K_ELEMS];
  __shared__ __attribute__((aligned(16))) _Float16 Vl[2][GEO::V_ELEMS];
  __shared__ __attribute__((aligned(16))) float KS[2][KT];
  __shared__ __attribute__((aligned(16))) float VS[2][KT];
  __shared__ __attribute__((aligned(16))) char stage[GEO::STAGE > 0 ? GEO::STAGE : 16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int c = lane & 15, g = lane >> 4;
  // uniform, kept in scalar registers (the compiler would otherwise treat
  // them, and everything derived from them, as varying across the lanes)
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Workgroup i of a launch runs on XCD i % 8.  When several query blocks
  // read the same K/V (one split of one KV head) and the (query block x
  // split, KV head) grid is a multiple of 8, logical block l = x + gx·y is
  // placed at i with l = (i % 8)·(n / 8) + i / 8, so that each XCD holds a
  // run of consecutive blocks -- the query blocks of one or two KV heads --
  // whose K/V tiles its L2 then serves to the rest of the run.
  int bx = blockIdx.x, by = blockIdx.y;
  {
    const int gx = gridDim.x, n = gx * gridDim.y;
    if (a.nqb > 1 && (n & 7) == 0) {
      const int i = bx + gx * by, l = (i & 7) * (n >> 3) + (i >> 3);
      by = l / gx;
      bx = l - by * gx;
    }
  }
  const int split = __builtin_amdgcn_readfirstlane(bx / a.nqb);
  const int qb = __builtin_amdgcn_readfirstlane(bx - split * a.nqb);
  const int h = __builtin_amdgcn_readfirstlane(by), b = blockIdx.z;
  const int64_t bh = (int64_t)b * a.Hkv + h;
  const int p0 = qb * a.block_rows;                     // the block's first row
  const int n_p = min(a.block_rows, a.L * a.G - p0);    // and its row count
  const int q_lo = __builtin_amdgcn_readfirstlane(p0 / a.G);  // its first and last query
  const int q_hi = __builtin_amdgcn_readfirstlane((p0 + n_p - 1) / a.G);
  const int P = (int)(a.T - a.L);  // cached tokens before the new ones
  const int t_blk = a.causal ? min((int)a.T, P + q_hi + 1) : (int)a.T;  // the block's keys end here
  // the wave's row tiles w and w + 8: how many exist (0, 1 or 2, uniform per
  // wave), and per lane its row in each (rows past the last repeat it) with
  // the row's query and query head
  const int nrt = 16 * w >= n_p ? 0 : 16 * (w + 8) >= n_p ? 1 : 2;
  const auto rows = [&](int cc, int (&prow)[2], int (&qr)[2], int (&hq)[2]) {
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      prow[rt] = 16 * (w + 8 * rt) + cc;
      const int p = p0 + min(prow[rt], n_p - 1);
      qr[rt] = p / a.G;
      hq[rt] = h * a.G + (p - qr[rt] * a.G);
    }
  };
  V8 qop[2][4];
  int qabs[2];  // the rows' query positions: all the main loop keeps of them
  {
    int prow[2], qr[2], hq[2];
    rows(c, prow, qr, hq);
    load_query<BF16>(qop, a, b, hq, qr, g);
    qabs[0] = P + qr[0];
    qabs[1] = P + qr[1];
  }
  // MM == 2: each row's bias row (element offset; the host keeps the extent
  // below 2^29 elements), read through a resource bounded by the extent
  uint32_t brow[2] = {0u, 0u};
  __amdgpu_buffer_rsrc_t rb = make_rsrc(a.bias.p, 0);
  if constexpr (MM == 2) {
    int prow[2], qr[2], hq[2];
    rows(c, prow, qr, hq);
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
      brow[rt] = (uint32_t)((int64_t)b * a.bias.sb + (int64_t)h * a.bias.skv +
                            (int64_t)(hq[rt] - h * a.G) * a.bias.sg + (int64_t)qr[rt] * a.bias.sl);
    rb = make_rsrc(a.bias.p, a.bias.extent * 4);
  }

  // a sliding window starts the scan at the first query's first visible key
  // (MM == 1: compiled in; without it the window is 0 and its terms vanish,
  // which keeps the quantized scans clear of register spills)
  const int window = MM == 1 ? a.window : 0;
  const int t_first = window > 0 ? max(0, P + q_lo - window + 1) / KT * KT : 0;
  // this workgroup's share of the keys, [lo, t_end): the split's range
  // (tile-aligned) within the query block's [t_first, t_blk); empty for some
  // splits.  A split that ends before t_blk ends on a tile boundary, so its
  // tiles are whole and t_end serves every load, mask and liveness test.
  const int64_t s_lo = a.split_lo + (int64_t)split * a.split_len;
  const int lo = __builtin_amdgcn_readfirstlane((int)max((int64_t)t_first, s_lo));
  const int t_end = __builtin_amdgcn_readfirstlane((int)min((int64_t)t_blk, s_lo + a.split_len));
  const auto stage_scales = [&](const TileRegs& R) {
    if (GEO::STAGE > 0 && 8 * tid < GEO::STAGE) *(v2i*)(stage + 8 * tid) = R.sc;
  };
  const auto convert = [&](const TileRegs& R, int bf, auto phase) {
    convert_tile<BF16, KF, VF, decltype(phase)::value>(R, Kl[bf], Vl[bf], KS[bf], VS[bf], stage, tid, a.q_mul);
  };
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  using P2 = std::integral_constant<int, 2>;
  const int qabs_lo = P + q_lo, qabs_hi = P + q_hi;
  // a unit needs the mask loop if it reaches the block's first diagonal, the
  // cache end, or (sliding window) lies before its last query's window start
  const auto needs_mask = [&](int tu) {
    return tu + 32 > qabs_lo || tu + 32 > t_end || (window > 0 && tu < qabs_hi - window + 1);
  };

  // The scan, compiled once per row-tile count NRT of the wave: a wave with
  // fewer tiles (the last block of a launch whose row count is not a
  // multiple of 256) runs the same pipeline with fewer matrix products, and
  // a wave with none only helps to load and dequantize the tiles.
  const auto scan = [&](auto nrt_c) {
    constexpr int NRT = decltype(nrt_c)::value;
    float m_use[2] = {0.f, 0.f}, thr[2] = {NEG_INF, NEG_INF}, l_run[2] = {0.f, 0.f};
    v4f acc[8][2];
#pragma unroll
    for (int n = 0; n < 8; ++n)
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) acc[n][rt] = (v4f){0.f, 0.f, 0.f, 0.f};

    // Prologue: tile lo into buffer 0 (all phases), the next tile's bytes in
    // flight.  Unconditional even for an empty range (lo >= t_end): every load
    // then fails its liveness test and reads nothing.
    TileRegs R;
    load_tile<KF, VF>(R, a, b, h, bh, lo, tid, t_end);
    stage_scales(R);
    __syncthreads();
    convert(R, 0, P0{});
    convert(R, 0, P1{});
    convert(R, 0, P2{});
    __syncthreads();
    if (lo + KT < t_end) load_tile<KF, VF>(R, a, b, h, bh, lo + KT, tid, t_end);

    // Software pipeline over 32-token units: the scores of unit u+1 are computed
    // on the matrix cores while the VALU runs the softmax of unit u.  A tile's
    // last unit is finished (softmax + P·V) at unit 0 of the next tile, from the
    // other buffer, which is refilled only at the end of that tile.
    v4f sc[2][2][2];    // scores of two units in flight: [unit parity][rt][j]
    bool pend = false;  // the previous unit awaits its softmax + P·V
    int pend_t = 0;
    int buf = 0;
    for (int t0 = lo; t0 < t_end; t0 += KT) {
      const bool more = t0 + KT < t_end;  // uniform
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int tu = t0 + 32 * u;
        const bool live = tu < t_end;
        if constexpr (NRT > 0) {
          if (live) {
            // the matrix-core bursts at raised wave priority: the SIMD's other
            // wave, in its softmax, fills the issue slots they leave (measured
            // 1.4% faster at 65,536 + 2,048 keys, 5% at 4,096 + 2,048)
            __builtin_amdgcn_s_setprio(1);
            qk_unit<BF16, NRT>(Kl[buf] + 32 * u * PF_KROW, qop, sc[u & 1], c, g);
            __builtin_amdgcn_s_setprio(0);
          }
          if (pend) {
            // the unit before: this tile's unit u - 1, or the previous tile's last
            const int pb_ = u == 0 ? buf ^ 1 : buf, po = u == 0 ? KT - 32 : 32 * (u - 1);
            softmax_pv_unit<VROW, GEO::VTR, EXACT, NRT, GEO::vpre(EXACT), MM == 2>(
                sc[(u + 1) & 1], Vl[pb_] + (GEO::VTR ? po * GEO::VPB : po), KS[pb_] + po, VS[pb_] + po, m_use, thr,
                l_run, acc, pend_t, t_end, qabs, a.causal, window, needs_mask(pend_t), c, g, rb, brow);
          }
        }
        pend = live;
        pend_t = tu;
      }
      if (more) {
        // The next tile, whose bytes had this whole tile to arrive, into the
        // other buffer: its scale bytes to the staging area, then (once every
        // wave has finished the unit that read the other buffer) the
        // dequantization; then the tile after next starts its way from HBM.
        stage_scales(R);
        __syncthreads();
        convert(R, buf ^ 1, P0{});
        convert(R, buf ^ 1, P1{});
        convert(R, buf ^ 1, P2{});
        if (t0 + 2 * KT < t_end) load_tile<KF, VF>(R, a, b, h, bh, t0 + 2 * KT, tid, t_end);
        __syncthreads();
        buf ^= 1;
      }
    }
    if constexpr (NRT > 0) {
      // still pending: the last tile's last unit (every unit of a tile is
      // visited, and a tile has an even number of units, so its scores are in sc[1])
      if (pend)
        softmax_pv_unit<VROW, GEO::VTR, EXACT, NRT, GEO::vpre(EXACT), MM == 2>(
            sc[1], Vl[buf] + GEO::vunit(U - 1), KS[buf] + KT - 32, VS[buf] + KT - 32, m_use, thr, l_run, acc,
            pend_t, t_end, qabs, a.causal, window, needs_mask(pend_t), c, g, rb, brow);

      // the rows again, from an opaque copy of the lane's column: recomputed
      // here rather than held in registers through the main loop
      int prow[2], qr[2], hq[2];
      {
        int cc = c;
        asm volatile("" : "+v"(cc));
        rows(cc, prow, qr, hq);
      }
      if (a.S > 1) {
        // ---------------- unnormalised partial of this split ----------------
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
          const float l = sum_xor32(sum_xor16(l_run[rt]));
          const float M = thr[rt] == NEG_INF ? NEG_INF : m_use[rt];  // -inf: no visible key in this split
          if (prow[rt] < n_p) {
            const int64_t row = (((int64_t)bh * a.S + split) * a.nqb + qb) * a.block_rows + prow[rt];
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
      for (int rt = 0; rt < NRT; ++rt) {
        float l = l_run[rt];
        l = sum_xor32(sum_xor16(l));
        float M = thr[rt] == NEG_INF ? NEG_INF : m_use[rt];  // -inf: no visible key
        if (a.sinks != nullptr) {
          const float sink = a.sinks[hq[rt]] * LOG2E;
          const float Mn = fmaxf(M, sink);
          const float f = M == NEG_INF ? 0.f : __builtin_amdgcn_exp2f(M - Mn);
          l = l * f + __builtin_amdgcn_exp2f(sink - Mn);
#pragma unroll
          for (int n = 0; n < 8; ++n) acc[n][rt] *= f;
        }
        const float inv = l > 0.f ? 1.f / l : 1.f;
        if (prow[rt] < n_p) {
          const int64_t o = (((int64_t)b * a.Hq + hq[rt]) * a.L + qr[rt]) * HEAD_DIM + 4 * g;
#pragma unroll
          for (int n = 0; n < 8; ++n) store_out4(a.out, o + 16 * n, acc[n][rt] * inv, a.out_dtype);
        }
      }
    }
  };
  if (nrt == 2) scan(std::integral_constant<int, 2>{});
  else if (nrt == 1) scan(std::integral_constant<int, 1>{});
  else scan(std::integral_constant<int, 0>{});
}

// Merge of the key splits (S > 1): one wavefront per (query, query head,
// batch); lane k owns the statistics of split k, the weights go through LDS,
// and lane l sums dims 2l, 2l + 1 over the splits.  The sink logit joins here.
// NR rounds of 16 split loads (S <= 16 NR), all issued before the first is
// used: one trip to memory, not one per round.
template <int NR>
__global__ __launch_bounds__(64) void prefill_merge_kernel(const PrefillArgs a) {
  static_assert(16 * NR <= PREFILL_MAX_SPLITS && PREFILL_MAX_SPLITS <= 64, "one split per lane");
  const int i = blockIdx.x, hq = blockIdx.y, b = blockIdx.z, lane = threadIdx.x;
  const int h = hq / a.G, p = i * a.G + (hq - h * a.G);  // the (query, head) row
  const int qb = p / a.block_rows, r = p - qb * a.block_rows;
  const int64_t bh = (int64_t)b * a.Hkv + h;
  const auto row = [&](int sp) { return ((bh * a.S + sp) * a.nqb + qb) * a.block_rows + r; };
  // every load first -- the splits' partial rows and their statistics -- so
  // that the merge waits for memory once (slots past the last split read its
  // row again and weigh it 0).  The rows of one (query, head) are a fixed
  // stride apart: each load takes its split's offset as a scalar, so the 64
  // addresses cost no vector instructions.
  const uint32_t step_b = (uint32_t)a.nqb * a.block_rows * HEAD_DIM * 4;  // bytes between consecutive splits' rows
  const uint32_t last_b = (uint32_t)(a.S - 1) * step_b;              // below 2^31 (prefill_plan)
  const __amdgpu_buffer_rsrc_t racc = make_rsrc(a.ws_acc + row(0) * HEAD_DIM, (int64_t)last_b + HEAD_DIM * 4);
  v2f x[16 * NR];
#pragma unroll
  for (int k = 0; k < 16 * NR; ++k)
    x[k] = __builtin_bit_cast(v2f, ld64<0>(racc, 8 * lane, (uint32_t)min(k, a.S - 1) * step_b));
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
  // split k's weight is lane k's f (0 past the last split), read as a scalar
  v2f acc = {0.f, 0.f};
#pragma unroll
  for (int k = 0; k < 16 * NR; ++k)
    acc += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, f), k)) * x[k];
  const float inv = z > 0.f ? 1.f / z : 1.f;
  store_out2(a.out, (((int64_t)b * a.Hq + hq) * a.L + i) * HEAD_DIM + 2 * lane, acc * inv, a.out_dtype);
}

PrefillPlan prefill_plan(const PrefillArgs& a, int requested) {
  PrefillPlan p{};
  const int rows = a.L * a.G;
  // A windowed launch's query blocks each scan at most window + block keys,
  // so a grid too small to fill the chip takes smaller blocks (128 or 64
  // rows; automatic or unsplit plans) before key splits, whose partials
  // (S x rows x 512 B) outweigh the window's K/V (bf16, 32 q / 4 kv heads:
  // a 512-token chunk over a 513-token window 36.7 -> 20.8 us with 64-row
  // blocks, a 1024-token chunk over a 4096-token window 178 -> 138 us with
  // 128-row blocks)
  p.block_rows = PF_ROWS;
  if (requested <= 1 && a.window > 0 && !prefill_few_fits(a))
    while (p.block_rows > 64 && (int64_t)((rows + p.block_rows - 1) / p.block_rows) * a.Hkv * a.B < 256)
      p.block_rows /= 2;
  p.nqb = (rows + p.block_rows - 1) / p.block_rows;
  const int kt = a.kv_bf16 ? PfGeom<FMT_BF, FMT_BF>::KT : PfGeom<8, 8>::KT;
  // keys any query block scans: from the first block's window start to T
  const int64_t P = a.T - a.L;
  const int64_t lo = a.window > 0 ? std::max<int64_t>(0, P - a.window + 1) / kt * kt : 0;
  const int64_t tiles = (a.T - lo + kt - 1) / kt;
  int S = requested;
  if (S <= 0) {
    // one workgroup per CU: split only a grid below half the chip, and keep
    // at least two tiles per split
    const int64_t nwg = (int64_t)p.nqb * a.Hkv * a.B;
    S = nwg >= 128 ? 1 : (int)std::min<int64_t>(PREFILL_MAX_SPLITS, (256 + nwg - 1) / nwg);
    if (!prefill_few_fits(a) && a.window == 0) {
      if (nwg >= 128 && nwg < 192) {
        // half to three quarters of the chip: a short prefix takes 128-row
        // blocks, a long one two key splits (int8, 32 q / 4 kv heads,
        // 1,024-token chunks after 0 / 1,024 / 2,048 / 4,096 / 8,192 tokens:
        // unsplit 55.0 / 99.7 / 141.7 / 224.8 / 312.9 us, two splits 59.7 /
        // 83.3 / 104.3 / 151.3 / 201.2, 128-row blocks 37.2 / 71.3 / 100.8 /
        // 161.2 / 240.0)
        if (P <= 2 * (int64_t)a.L) {
          p.block_rows = PF_ROWS / 2;
          p.nqb = (rows + p.block_rows - 1) / p.block_rows;
        } else {
          S = 2;
        }
      } else if (nwg < 128) {
        // splits of at least two tiles cannot fill the chip: smaller blocks
        // as well, while the grid stays one round (128 queries after 1,024
        // tokens, int8: 4 splits 31.5 us, 4 splits of 64-row blocks 20.9;
        // a bf16 cache's 9 splits of 128-row blocks, 288 workgroups, were
        // slower than 144)
        const int64_t s_max = std::max<int64_t>(1, std::min<int64_t>(S, tiles / 2));
        while (p.block_rows > 64 && (int64_t)p.nqb * a.Hkv * a.B * s_max < 192 &&
               (int64_t)((rows + p.block_rows / 2 - 1) / (p.block_rows / 2)) * a.Hkv * a.B * s_max <= 256) {
          p.block_rows /= 2;
          p.nqb = (rows + p.block_rows - 1) / p.block_rows;
        }
      }
    }
    // the streaming kernel's row groups are workgroups of their own: as many
    // splits as fill the chip once, so that every workgroup runs beside its
    // unit's other row groups (20 queries x 8 heads over 32K keys: 16 splits
    // 31.1 us, 24 and 32 splits 42.2 and 40.5 us)
    if (prefill_few_fits(a) && prefill_few_groups(a) > 1) {
      const int64_t g = (int64_t)prefill_few_groups(a) * a.Hkv * a.B;
      S = (int)std::max<int64_t>(1, std::min<int64_t>(PREFILL_MAX_SPLITS, 256 / g));
    }
    S = (int)std::min<int64_t>(S, std::max<int64_t>(1, tiles / 2));
  }
  S = std::max(1, std::min(S, PREFILL_MAX_SPLITS));
  S = (int)std::min<int64_t>(S, std::max<int64_t>(1, tiles));
  // the merge addresses one row's partials with 32-bit offsets from its first
  // split: (S - 1) strides of nqb * block_rows rows of 512 bytes stay below 2^31
  const int64_t stride_b = (int64_t)p.nqb * p.block_rows * HEAD_DIM * 4;
  S = (int)std::min<int64_t>(S, 1 + (((int64_t)1 << 31) - 1 - HEAD_DIM * 4) / stride_b);
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

size_t prefill_ws_bytes(int B, int Hkv, int64_t head_rows, int S) {
  if (S <= 1) return 0;
  const size_t rows = (size_t)B * Hkv * S * head_rows;
  return rows * HEAD_DIM * 4 + rows * 2 * 4;
}

template <bool BF16, bool EXACT, int MM>
static void launch_quantized(const PrefillArgs& a, dim3 grid, dim3 block, hipStream_t stream) {
  const int kf = a.k_fmt, vf = a.v_fmt;
  if (kf == 8 && vf == 8) hipLaunchKernelGGL((prefill_kernel<BF16, 8, 8, EXACT, MM>), grid, block, 0, stream, a);
  else if (kf == 8 && vf == 4) hipLaunchKernelGGL((prefill_kernel<BF16, 8, 4, EXACT, MM>), grid, block, 0, stream, a);
  else if (kf == 4 && vf == 8) hipLaunchKernelGGL((prefill_kernel<BF16, 4, 8, EXACT, MM>), grid, block, 0, stream, a);
  else if (kf == 4 && vf == 4) hipLaunchKernelGGL((prefill_kernel<BF16, 4, 4, EXACT, MM>), grid, block, 0, stream, a);
  else if (kf == FMT_A8) hipLaunchKernelGGL((prefill_kernel<BF16, FMT_A8, FMT_A4, EXACT, MM>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((prefill_kernel<BF16, FMT_A8H, FMT_A4H, EXACT, MM>), grid, block, 0, stream, a);
}

// The bf16 cache (ring windows) always takes the window at run time; the
// quantized formats have a variant with it and one without.  A bias (mask
// array) takes its own variants, always with the exact P·V: a mask may leave
// any row a few visible keys.
template <bool BF16, bool EXACT>
static void launch_formats(const PrefillArgs& a, dim3 grid, dim3 block, hipStream_t stream) {
  if (a.bias.p != nullptr) {
    if (a.k_fmt == FMT_BF) hipLaunchKernelGGL((prefill_kernel<BF16, FMT_BF, FMT_BF, true, 2>), grid, block, 0, stream, a);
    else launch_quantized<BF16, true, 2>(a, grid, block, stream);
  } else if (a.k_fmt == FMT_BF) {
    hipLaunchKernelGGL((prefill_kernel<BF16, FMT_BF, FMT_BF, EXACT, 1>), grid, block, 0, stream, a);
  } else if (a.window > 0) {
    launch_quantized<BF16, EXACT, 1>(a, grid, block, stream);
  } else {
    launch_quantized<BF16, EXACT, 0>(a, grid, block, stream);
  }
}

// Fewest keys any query row of the launch sees: the first row's causal
// prefix (and at most the window), or all T keys without a causal mask.
static int64_t fewest_visible_keys(const PrefillArgs& a) {
  int64_t n = a.causal ? a.T - a.L + 1 : a.T;
  if (a.window > 0 && a.window < n) n = a.window;
  return n;
}

hipError_t launch_prefill(const PrefillArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)(a.nqb * a.S), a.Hkv, a.B), block(512);
  const bool exact = fewest_visible_keys(a) < EXACT_PV_BELOW;
  if (prefill_few_fits(a)) {
    const hipError_t e = launch_prefill_few(a, stream);
    if (e != hipSuccess) return e;
  } else if (a.q_dtype == DT_BF16) {
    if (exact) launch_formats<true, true>(a, grid, block, stream);
    else launch_formats<true, false>(a, grid, block, stream);
  } else {
    if (exact) launch_formats<false, true>(a, grid, block, stream);
    else launch_formats<false, false>(a, grid, block, stream);
  }
  if (a.S > 1) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const dim3 grid((unsigned)a.L, a.Hq, a.B), block(64);
    if (a.S <= 16) hipLaunchKernelGGL(prefill_merge_kernel<1>, grid, block, 0, stream, a);
    else if (a.S <= 32) hipLaunchKernelGGL(prefill_merge_kernel<2>, grid, block, 0, stream, a);
    else if (a.S <= 48) hipLaunchKernelGGL(prefill_merge_kernel<3>, grid, block, 0, stream, a);
    else hipLaunchKernelGGL(prefill_merge_kernel<4>, grid, block, 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace rec
