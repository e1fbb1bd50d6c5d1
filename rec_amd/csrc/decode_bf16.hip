// Split-K flash decode over a bf16 KV cache (gfx950): the reference's
// production cache format.
//
// Restates, for bf16 K/V held token-major ([token][128] rows, the layout of
// KVStorage / FixedKVCache, engine/src/rec_mlx/cache.py:30-150):
//   * the attention of Attention.__call__ over a FixedKVCache
//     (engine/src/rec_mlx/model.py:204-211, scaled_dot_product_attention with the
//     per-head sink logit), which the reference's fused decoder runs as the
//     bf16 split-K partial of engine/src/rec_mlx/kernels/megakernel.py:619-693;
//   * the write of the new token into the storage (cache.py:30-45, :97-119),
//     fused: the split that owns the newest token writes it first.
// Partials use the layout of the quantized decode, and rec_decode_merge /
// the merge kernel combine them.
//
// Work decomposition: as the quantized decode — grid (splits, Hkv, B), 4
// wavefronts, wave w takes 32-token chunks w, w+4, ..., a 2-deep ring of raw
// buffer loads (chunks past the wave's last one load through an empty
// resource and only their compute is skipped).  Every load instruction reads
// 1 KB of contiguous cache (four 256-byte rows, 16 bytes per lane): loads
// shaped as the MFMA operands want them (64 bytes of each of 16 rows per
// instruction) streamed at 5.5 TB/s where contiguous ones reach 6.5, and this
// kernel is bound by its loads, so each wave stages its chunk's K and V rows
// in LDS and reads the operands from there.
//
// Q·Kᵀ on v_mfma_f32_16x16x32_bf16: A = 16 K rows x 32 dims (ds_read_b128 of
// the staged rows, a 272-byte pitch keeping 8 consecutive rows on distinct
// banks), B = the scaled query split into bf16 high and low parts that fill
// the 16 columns (columns 0-7 = high parts of heads 0-7, 8-15 = low parts: 16
// significant bits), recombined with one DPP row rotation.
//
// P·V on the same MFMA.  The A operand is Vᵀ (16 dims x 32 tokens) while the
// cache holds V token-major: the staged V rows sit at the block positions of
// the quantized layout, which puts lane group g's tokens at rows 8g .. 8g+7,
// and the operand is read back with ds_read_b64_tr_b16: in a group of 16 lanes, lane 4a+b receives element b of
// the 8-byte rows addressed by lanes 4k+a (k = 0..3), so lanes addressing rows
// 8g+k, dims 16n+4a hand lane c dim 16n+c of four consecutive rows.  The
// probabilities split the same way (columns 0-7 bf16(p), 8-15 the bf16
// remainder), and the two column halves of the result are added at the end.
#include "kernels.h"

namespace rec {
namespace {

constexpr int BCH = 32;        // tokens per chunk
constexpr int ROWB = 256;      // bytes per K/V row (128 bf16)
constexpr int VPITCH = 288;    // LDS bytes per staged V row: 256 + 32 keeps the transposed reads conflict-free
constexpr int KPITCH = 272;    // LDS bytes per staged K row: 256 + 16

constexpr int BW = 4;          // wavefronts per workgroup
constexpr int BL_QOP = 0;                             // 4 k-steps x 64 lanes x 16 B
constexpr int BL_PART = 4096;                         // wave partials: 4 x 8 x 128 floats
constexpr int BL_PSTAT = BL_PART + BW * 8 * 128 * 4;  // 4 x 8 x (m, l)
constexpr int BL_V = BL_PSTAT + BW * 8 * 8;           // per wave: 32 rows x VPITCH
constexpr int BL_K = BL_V + BW * BCH * VPITCH;        // per wave: 32 rows x KPITCH
constexpr int BL_BYTES = BL_K + BW * BCH * KPITCH;

typedef __bf16 v4bf __attribute__((ext_vector_type(4)));

// One chunk as it arrives from HBM: load i is bytes [1024 i, 1024 i + 1024)
// of the chunk's K (V) rows, lane (c, kg) holding token 4i + kg, dims 8c .. 8c+7.
struct BChunk {
  v4i k[8];
  v4i v[8];
};

struct BState {
  float m, l;
  v4f acc[8];  // columns 0-7: P_hi · V, columns 8-15: P_lo · V
};

__device__ __forceinline__ void load_bchunk(BChunk& R, __amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv,
                                            __amdgpu_buffer_rsrc_t none, bool ok, uint32_t blk, uint32_t loff) {
  const __amdgpu_buffer_rsrc_t a = ok ? rk : none, b = ok ? rv : none;
#pragma unroll
  for (int i = 0; i < 8; ++i) R.k[i] = ld128(a, loff + i * 1024, blk * BCH * ROWB);
#pragma unroll
  for (int i = 0; i < 8; ++i) R.v[i] = ld128(b, loff + i * 1024, blk * BCH * ROWB);
}

// Stage a chunk's rows in the wave's LDS rows: K token t at row t, V token t
// at row block_pos(t).  new_row >= 0: that row is the token this launch
// writes, and its bf16 values (kw, vw: this lane's two dims of K and V)
// replace what the load returned -- the write to memory need not land before
// the chunk's load.
__device__ __forceinline__ void stage_bchunk(const BChunk& R, int lane, char* vl, char* kl, int new_row, uint32_t kw,
                                             uint32_t vw) {
  const int c = lane & 15, kg = lane >> 4;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    *(v4i*)(kl + (4 * i + kg) * KPITCH + 16 * c) = R.k[i];
    *(v4i*)(vl + block_pos(4 * i + kg) * VPITCH + 16 * c) = R.v[i];
  }
  if (__builtin_expect(new_row >= 0, 0)) {
    *(uint32_t*)(kl + new_row * KPITCH + 4 * lane) = kw;
    *(uint32_t*)(vl + block_pos(new_row) * VPITCH + 4 * lane) = vw;
  }
}

// The Vᵀ operands of a staged chunk (ds_read_b64_tr_b16, see the file header).
__device__ __forceinline__ void read_vt(v8bf* va, int lane, const char* vl) {
  const int kg = lane >> 4, sk = (lane & 15) >> 2, sa = lane & 3;  // lane addresses row 8kg + sk (+4), dims 16n + 4sa
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    typedef __attribute__((address_space(3))) v4bf lds_v4bf;
    const char* base = vl + (8 * kg + sk) * VPITCH + (16 * n + 4 * sa) * 2;
    const v4bf r0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_v4bf*)(base));
    const v4bf r1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_v4bf*)(base + 4 * VPITCH));
    va[n] = (v8bf){r0[0], r0[1], r0[2], r0[3], r1[0], r1[1], r1[2], r1[3]};
  }
}

// One staged chunk: Q·Kᵀ, online softmax, P·V.  MASK: bz holds the bias of
// the lane's tokens 16j + 4kg + i (natural-log units, -inf drops a token).
template <bool MASK>
__device__ __forceinline__ void compute_bchunk(BState& st, const v8bf* qop, int valid, int lane, char* vl, char* kl,
                                               const v4i* bz) {
  const int c = lane & 15, kg = lane >> 4;
  wave_lds_sync();

  // ---------------- scores (log2 domain: the query carries scale * log2 e) ----------------
  // every LDS operand read of the chunk first -- the eight K operands, then
  // the sixteen transposed V reads -- so that the matrix products wait for
  // the LDS once and the V reads arrive behind the Q·Kᵀ and the softmax
  v8bf ka[2][4], va[8];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) ka[j][ks] = *(const v8bf*)(kl + (16 * j + c) * KPITCH + 64 * ks + 16 * kg);
  read_vt(va, lane, vl);
  __builtin_amdgcn_sched_barrier(0);
  float s[8];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    v4f d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[j][ks], qop[ks], d, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) s[4 * j + i] = d[i] + dpp_ror8f(d[i]);  // high part + low part
  }
  if constexpr (MASK) {
#pragma unroll
    for (int idx = 0; idx < 8; ++idx) {
      const int w = bz[idx >> 2][idx & 3];  // a copy: a bit_cast of a vector subscript reads element 0
      s[idx] = __builtin_fmaf(__builtin_bit_cast(float, w), LOG2E, s[idx]);
    }
  }
  // tail chunk: tokens past the split end (rare: without the hint the
  // compiler turns this into compares and selects on every chunk)
  if (__builtin_expect(valid < BCH, 0)) {
#pragma unroll
    for (int idx = 0; idx < 8; ++idx)
      if (16 * (idx >> 2) + 4 * kg + (idx & 3) >= valid) s[idx] = NEG_INF;
  }

  // ---------------- online softmax (lazy running max, RESCALE_GAP) ----------------
  float cmax = s[0];
#pragma unroll
  for (int idx = 1; idx < 8; ++idx) cmax = maxp(cmax, s[idx]);
  if (__ballot(cmax > st.m + RESCALE_GAP)) {
    cmax = max_xor32(max_xor16(cmax));
    const float m_new = fmaxf(st.m, cmax);
    // (MASK: a head whose every score so far is -inf keeps m = -inf, zero sums)
    const float factor = MASK && st.m == NEG_INF ? 0.f : __builtin_amdgcn_exp2f(st.m - m_new);
    st.l *= factor;
#pragma unroll
    for (int n = 0; n < 8; ++n) st.acc[n] *= factor;
    st.m = m_new;
  }
  // P split into bf16 high (columns 0-7) and low (8-15) parts, position order
  v8bf pb;
#pragma unroll
  for (int idx = 0; idx < 8; ++idx) {
    const float p = __builtin_amdgcn_exp2f(s[idx] - (MASK && st.m == NEG_INF ? 0.f : st.m));
    st.l += p;
    const __bf16 hi = (__bf16)p;
    pb[idx] = c < 8 ? hi : (__bf16)(p - (float)hi);
  }

  // ---------------- P·V: the Vᵀ operands read above ----------------
#pragma unroll
  for (int n = 0; n < 8; ++n) st.acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[n], pb, st.acc[n], 0, 0, 0);
  wave_lds_sync();  // the next chunk's staging overwrites these rows (K and V)
}

// This lane's two dims (2 lane, 2 lane + 1) of the new token's row, rounded to bf16 and packed.
__device__ __forceinline__ uint32_t bf16_row_pair(const RowSrc& src, int b, int h, int lane) {
  float x0, x1;
  load2_as_float(src, row_base(src, b, h, 0) + 2 * lane, x0, x1);
  const __bf16 h0 = (__bf16)x0, h1 = (__bf16)x1;
  return (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
}

template <bool MASK>
__global__ __launch_bounds__(256) void decode_bf16_kernel(const DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[BL_BYTES];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, kg = lane >> 4;
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int64_t bh = (int64_t)b * a.Hkv + h;
  const bool fused = a.knew.p != nullptr;
  const bool tail = fused && split == a.S - 1;
  int t_begin, t_end;
  if (tail) {
    t_begin = a.t_split_end;
    t_end = (int)a.T;
  } else {
    t_begin = split * a.span;
    t_end = t_begin + a.span < a.t_split_end ? t_begin + a.span : a.t_split_end;
  }

  const __bf16* kbase = (const __bf16*)a.kq + (int64_t)b * a.k_sb + (int64_t)h * a.k_sh;
  const __bf16* vbase = (const __bf16*)a.vq + (int64_t)b * a.v_sb + (int64_t)h * a.v_sh;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase, a.T * ROWB), rv = make_rsrc(vbase, a.T * ROWB);
  const __amdgpu_buffer_rsrc_t none = make_rsrc(kbase, 0);

  // Query first, then the first chunks, then (fused) the new token's row:
  // nothing waits for anything before the loads are out.
  const int hh = tid >> 5, d0 = (tid & 31) * 4;
  const int hq_ld = h * a.G + (hh < a.G ? hh : 0);
  const int64_t qi = (int64_t)b * a.q_sb + (int64_t)hq_ld * a.q_sh + d0;
  const int es = a.q_dtype == DT_F32 ? 4 : 2;
  const char* qp = (const char*)a.q + qi * es;
  const v2i qw0 = *(const v2i*)qp;
  const v2i qw1 = *(const v2i*)(qp + (es == 4 ? 8 : 0));

  constexpr int NBUF = 2;  // chunks in flight per wave
  const int n_split = (t_end - t_begin + BCH - 1) / BCH;
  const int n_w = n_split > wave ? (n_split - wave + BW - 1) / BW : 0;
  const int blk0 = t_begin / BCH + wave;
  const uint32_t loff = (uint32_t)(16 * lane);
  BChunk buf[NBUF];
  load_bchunk(buf[0], rk, rv, none, 0 < n_w, blk0, loff);
  // MASK: the bias row of this lane's head (column c, head c mod 8), two
  // 16-byte runs per chunk, loaded with the chunk into a ring of its own
  v4i bz[NBUF][2];
  __amdgpu_buffer_rsrc_t rb = none;
  uint32_t boff = 0;
  if constexpr (MASK) {
    const int64_t base = (int64_t)b * a.bias.sb + (int64_t)h * a.bias.skv;
    rb = make_rsrc(a.bias.p + base, (a.bias.extent - base) * 4);
    const int gq = (c & 7) < a.G ? (c & 7) : 0;
    boff = (uint32_t)(((int64_t)gq * a.bias.sg + 4 * kg) * 4);
  }
  const auto load_bias = [&](v4i(&z)[2], bool ok, int blk) {
    if constexpr (MASK) {
      const __amdgpu_buffer_rsrc_t r = ok ? rb : none;
      const uint32_t t0 = (uint32_t)blk * BCH * 4;
      z[0] = ld128<0>(r, boff + t0, 0);
      z[1] = ld128<0>(r, boff + t0 + 64, 0);
    }
  };
  load_bias(bz[0], 0 < n_w, blk0);

  // Fused write of the newest token (position new_pos: T-1, or a ring slot)
  // by the wave whose chunk holds it, in the split whose range holds it:
  // ranges start on chunk boundaries, so no other wave or split reads that
  // position.  The wave puts the token's bf16 values into its staged chunk
  // (stage_bchunk) and stores them for later steps: nothing waits for the
  // store, and the chunk's own load of that row (old or new bytes) is
  // overwritten in LDS.
  const bool writes = fused && t_begin <= a.new_pos && a.new_pos < t_end;
  const int new_chunk = writes ? (int)(a.new_pos / BCH) - t_begin / BCH : -1;  // chunk within the split
  const bool owner = writes && new_chunk % BW == wave;
  const int new_step = owner ? new_chunk / BW : -1;  // this wave's step that holds the new token
  const int new_row = writes ? (int)(a.new_pos % BCH) : -1;
  uint32_t knew_w = 0, vnew_w = 0;
  if (owner) {
    knew_w = bf16_row_pair(a.knew, b, h, lane);
    vnew_w = bf16_row_pair(a.vnew, b, h, lane);
  }

  {
    __bf16* qop = (__bf16*)(smem + BL_QOP);
    if (tid < 256) {
      const v4i raw = {qw0[0], qw0[1], qw1[0], qw1[1]};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rk_ = raw[i];  // copy first: bit_cast of a vector subscript reads lane 0 in this clang
        const uint32_t w = (uint32_t)raw[i >> 1];
        const uint32_t bits = (i & 1) ? (w >> 16) : (w & 0xffffu);
        float x = a.q_dtype == DT_F32 ? __builtin_bit_cast(float, rk_)
                                      : (a.q_dtype == DT_F16 ? half_bits_to_float(bits)
                                                             : __builtin_bit_cast(float, bits << 16));
        x *= hh < a.G ? a.q_mul : 0.f;
        const __bf16 hi = (__bf16)x, lo = (__bf16)(x - (float)hi);
        const int d = d0 + i, ks = d >> 5, g = (d >> 3) & 3, jj = d & 7;
        qop[(ks * 64 + g * 16 + hh) * 8 + jj] = hi;
        qop[(ks * 64 + g * 16 + hh + 8) * 8 + jj] = lo;
      }
    }
  }
  __syncthreads();
  if (owner) {
    *(uint32_t*)((__bf16*)a.kq + (int64_t)b * a.k_sb + (int64_t)h * a.k_sh + a.new_pos * HEAD_DIM + 2 * lane) = knew_w;
    *(uint32_t*)((__bf16*)a.vq + (int64_t)b * a.v_sb + (int64_t)h * a.v_sh + a.new_pos * HEAD_DIM + 2 * lane) = vnew_w;
  }
  v8bf qop[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) qop[ks] = ((const v8bf*)(smem + BL_QOP))[ks * 64 + lane];

  BState st;
  st.m = NEG_INF;
  st.l = 0.f;
#pragma unroll
  for (int n = 0; n < 8; ++n) st.acc[n] = (v4f){0.f, 0.f, 0.f, 0.f};
  char* vl = smem + BL_V + wave * BCH * VPITCH;
  char* kl = smem + BL_K + wave * BCH * KPITCH;

  // Ring as in the quantized decode: step i loads chunk i+1, then stages and
  // computes chunk i (its freed registers take the operands); padded to whole
  // revolutions, padding steps load through an empty resource (no load sits
  // under a branch) and only their staging and compute are skipped.
  const int n_pad = (n_w + NBUF - 1) / NBUF * NBUF;
  for (int i0 = 0; i0 < n_pad; i0 += NBUF) {
#pragma unroll
    for (int j = 0; j < NBUF; ++j) {
      const int i = i0 + j;
      load_bchunk(buf[(j + 1) % NBUF], rk, rv, none, i + 1 < n_w, blk0 + BW * (i + 1), loff);
      load_bias(bz[(j + 1) % NBUF], i + 1 < n_w, blk0 + BW * (i + 1));
      if (i < n_w) {
        stage_bchunk(buf[j], lane, vl, kl, i == new_step ? new_row : -1, knew_w, vnew_w);
        compute_bchunk<MASK>(st, qop, t_end - (blk0 + BW * i) * BCH, lane, vl, kl, bz[j]);
      }
    }
  }

  // ---------------- wave partial -> LDS (columns c and c+8 summed) ----------------
  st.l = sum_xor32(sum_xor16(st.l));
  float* part = (float*)(smem + BL_PART);
  float* pstat = (float*)(smem + BL_PSTAT);
#pragma unroll
  for (int n = 0; n < 8; ++n)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = st.acc[n][i] + dpp_ror8f(st.acc[n][i]);
      if (c < 8 && c < a.G) part[(wave * 8 + c) * HEAD_DIM + 16 * n + 4 * kg + i] = v;
    }
  if (c < 8 && c < a.G && kg == 0) {
    pstat[(wave * 8 + c) * 2 + 0] = st.m;
    pstat[(wave * 8 + c) * 2 + 1] = st.l;
  }
  __syncthreads();

  // ---------------- workgroup partial (or the output when S == 1) ----------------
  if (hh < a.G) {
    float mw[BW], M = NEG_INF;
#pragma unroll
    for (int w = 0; w < BW; ++w) {
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
    for (int w = 0; w < BW; ++w) {
      const float f = (mw[w] == NEG_INF || M == NEG_INF) ? 0.f : __builtin_amdgcn_exp2f(mw[w] - M);
      acc4 += f * *(const v4f*)(part + (w * 8 + hh) * HEAD_DIM + d0);
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

// Bulk write of L new rows into bf16 K/V storage (FixedKVCache.update_and_fetch's
// write, cache.py:97-119): one wavefront per (row, K or V), two elements per lane.
__global__ __launch_bounds__(256) void write_bf16_kernel(const AppendArgs a, int64_t k_sb, int64_t k_sh,
                                                         int64_t v_sb, int64_t v_sh) {
  const int lane = threadIdx.x & 63;
  const int64_t total = (int64_t)a.B * a.Hkv * a.L;
  const bool isv = blockIdx.y == 1;
  const RowSrc& src = isv ? a.v : a.k;
  for (int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); unit < total; unit += (int64_t)gridDim.x * 4) {
    const int64_t bh = unit / a.L, u = unit % a.L;
    const int b = (int)(bh / a.Hkv), h = (int)(bh % a.Hkv);
    float x0, x1;
    load2_as_float(src, row_base(src, b, h, (int)u) + 2 * lane, x0, x1);
    const __bf16 h0 = (__bf16)x0, h1 = (__bf16)x1;
    const uint32_t w = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
    __bf16* dst = (__bf16*)(isv ? a.vq : a.kq) + (int64_t)b * (isv ? v_sb : k_sb) + (int64_t)h * (isv ? v_sh : k_sh);
    *(uint32_t*)(dst + (a.offset + u) * HEAD_DIM + 2 * lane) = w;
  }
}

// The keys (values) a chunk attends over in a sliding-window ring
// (FixedSlidingKVCache.update_and_fetch, cache.py:227-247): the n held tokens
// in sequence order -- token i at ring slot (head + i) mod capacity -- then
// the L new rows rounded to bf16, into one (B, Hkv, n + L, 128) tensor.  One
// wavefront per (row, K or V), two elements per lane, as write_bf16_kernel.
// With place, chunk rows j >= keep_from (sequence position a.offset + j) also
// go to their ring slots.  A slot that holds a token of the window is
// rewritten by the wavefront that reads it, after its read: no other
// wavefront touches it, so the launch needs no ordering between them.
__global__ __launch_bounds__(256) void ring_join_kernel(const AppendArgs a, __bf16* rk, __bf16* rv,
                                                        int64_t rk_sb, int64_t rk_sh, int64_t rv_sb, int64_t rv_sh,
                                                        int64_t head, int64_t n, int64_t keep_from, bool place,
                                                        __bf16* ok, __bf16* ov) {
  const int lane = threadIdx.x & 63;
  const int64_t rows = n + a.L;
  const int64_t total = (int64_t)a.B * a.Hkv * rows;
  const bool isv = blockIdx.y == 1;
  const RowSrc& src = isv ? a.v : a.k;
  for (int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); unit < total; unit += (int64_t)gridDim.x * 4) {
    const int64_t bh = unit / rows, u = unit % rows;
    const int b = (int)(bh / a.Hkv), h = (int)(bh % a.Hkv);
    __bf16* ring = isv ? rv + (int64_t)b * rv_sb + (int64_t)h * rv_sh : rk + (int64_t)b * rk_sb + (int64_t)h * rk_sh;
    const auto chunk_row = [&](int64_t j) {
      float x0, x1;
      load2_as_float(src, row_base(src, b, h, (int)j) + 2 * lane, x0, x1);
      const __bf16 h0 = (__bf16)x0, h1 = (__bf16)x1;
      return (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
    };
    uint32_t* dst = (uint32_t*)((isv ? ov : ok) + unit * HEAD_DIM + 2 * lane);
    if (u < n) {
      const int64_t slot = (head + u) % a.cap;
      uint32_t* rs = (uint32_t*)(ring + slot * HEAD_DIM + 2 * lane);
      *dst = *rs;  // the old token's bytes are stored before the slot is rewritten
      if (place) {
        // the chunk row landing on this slot, if any: j >= keep_from with
        // a.offset + j = slot (mod capacity)
        const int64_t j = keep_from + ((slot - (a.offset + keep_from)) % a.cap + a.cap) % a.cap;
        if (j < a.L) *rs = chunk_row(j);
      }
    } else {
      const int64_t j = u - n;
      const uint32_t w = chunk_row(j);
      *dst = w;
      if (place && j >= keep_from) {
        const int64_t slot = (a.offset + j) % a.cap;
        if ((slot - head + a.cap) % a.cap >= n) *(uint32_t*)(ring + slot * HEAD_DIM + 2 * lane) = w;  // not held
      }
    }
  }
}

}  // namespace

hipError_t launch_ring_join_bf16(const AppendArgs& a, void* rk, void* rv, int64_t rk_sb, int64_t rk_sh,
                                 int64_t rv_sb, int64_t rv_sh, int64_t head, int64_t n, int64_t keep_from, bool place,
                                 void* ok, void* ov, hipStream_t stream) {
  const int64_t rows = (int64_t)a.B * a.Hkv * (n + a.L);
  const int64_t wgs = (rows + 3) / 4;
  const unsigned grid_x = (unsigned)(wgs < (1 << 20) ? (wgs > 0 ? wgs : 1) : (1 << 20));  // the kernel strides over rows
  hipLaunchKernelGGL(ring_join_kernel, dim3(grid_x, 2), dim3(256), 0, stream, a, (__bf16*)rk, (__bf16*)rv, rk_sb,
                     rk_sh, rv_sb, rv_sh, head, n, keep_from, place, (__bf16*)ok, (__bf16*)ov);
  return hipGetLastError();
}

hipError_t launch_decode_bf16(const DecodeArgs& a, hipStream_t stream) {
  if (a.bias.p != nullptr)
    hipLaunchKernelGGL(decode_bf16_kernel<true>, dim3(a.S, a.Hkv, a.B), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(decode_bf16_kernel<false>, dim3(a.S, a.Hkv, a.B), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_write_bf16(const AppendArgs& a, int64_t k_sb, int64_t k_sh, int64_t v_sb, int64_t v_sh,
                             hipStream_t stream) {
  const int64_t rows = (int64_t)a.B * a.Hkv * a.L;
  const int64_t wgs = (rows + 3) / 4;
  const unsigned grid_x = (unsigned)(wgs < (1 << 20) ? (wgs > 0 ? wgs : 1) : (1 << 20));  // the kernel strides over rows
  hipLaunchKernelGGL(write_bf16_kernel, dim3(grid_x, 2), dim3(256), 0, stream, a, k_sb, k_sh, v_sb,
                     v_sh);
  return hipGetLastError();
}

}  // namespace rec
