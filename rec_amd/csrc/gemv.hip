// int4 group-64 GEMV of the decoder's projections on bf16 MFMA.
//
// Restates q4 / dot16 of engine/src/rec_mlx/kernels/megakernel.py:161-232:
// y[m][r] = Σ_g ( s[r][g] · Σ_{k∈g} q[r][k] x[m][k] + b[r][g] · Σ_{k∈g} x[m][k] )
// for an MLX affine 4-bit matrix (group 64: uint32 words of 8 codes, code e
// at bits 4e; bf16 scales and biases per (row, group)), bf16 x and a bf16 (or
// fp32) result.  The weights are repacked once (q4_pack_kernel) into records
// that one wavefront streams linearly.
//
// Packed layout: per 16-row tile and 128-element span, one 1152-byte record
//   [64 lanes][16 B]  codes: lane (r, kq) holds row r, elements 32kq .. 32kq+31
//                     of the span (four MLX words, unchanged)
//   [4 rg][2 gs][16 B] row group rg, group 2·span+gs: scales of rows 4rg..4rg+3
//                     (4 x bf16), then their biases (4 x bf16)
// Records are ordered [tile][span]; rows past N are zero.
//
// Arithmetic: the codes enter a bf16 MFMA 16x16x32 as 128 + q (exact: the
// nibble under the bf16 exponent of 128), x as bf16, products exact in fp32.
// The B operand's 16 columns are (vector m, group half gs): a column only
// holds x for the elements of its group, so one MFMA yields separate sums
// D = Σ (128 + q) x for the two groups of a span, and
// y += s·D + (b − 128 s)·X with X = Σ x over the group.
#include "kernels.h"

namespace rec {

namespace {

constexpr int GV_WAVES = 4;        // waves per workgroup (more for matrices of few tiles)
constexpr int GV_SPAN = 128;         // elements per span
constexpr int GV_REC = 1024 + 128;   // bytes per (tile, span) record
constexpr int GV_ZERO = 256;         // zero bytes read by B lanes without data

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

// bf16 round-to-nearest-even of a finite or infinite float (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

}  // namespace

// One workgroup of 64 threads per (tile, span) record.
__global__ __launch_bounds__(64) void q4_pack_kernel(const Q4PackArgs a) {
  const int l = threadIdx.x;
  const int64_t tile = blockIdx.y, span = blockIdx.x;
  const int64_t S = a.K / GV_SPAN, words = a.K / 8, groups = a.K / 64;
  uint8_t* rec = a.packed + (tile * S + span) * GV_REC;
  {
    const int64_t row = tile * 16 + (l & 15);
    v4i w = {0, 0, 0, 0};
    if (row < a.N) {
      const uint32_t* src = a.w + row * words + span * 16 + 4 * (l >> 4);
      w = (v4i){(int)src[0], (int)src[1], (int)src[2], (int)src[3]};
    }
    *(v4i*)(rec + 16 * l) = w;
  }
  if (l < 8) {
    const int rg = l >> 1, gs = l & 1;
    const int64_t g = 2 * span + gs;
    uint16_t v[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t row = tile * 16 + 4 * rg + i;
      v[i] = row < a.N ? a.scales[row * groups + g] : 0;
      v[4 + i] = row < a.N ? a.biases[row * groups + g] : 0;
    }
    v4i o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (int)(v[2 * i] | ((uint32_t)v[2 * i + 1] << 16));
    *(v4i*)(rec + 1024 + 16 * l) = o;
  }
}

// LDS: [M][S][4 slabs][4 kq][8 bf16] permuted x, a zero block, [M][K/64]
// group sums, and the waves' partial results ([4 waves][64 lanes][4 floats]).
__host__ __device__ size_t q4_gemv_red_offset(int M, int64_t K) {
  return ((size_t)M * K * 2 + GV_ZERO + (size_t)M * (K / 64) * 4 + 15) & ~(size_t)15;
}

static size_t lds_bytes_nw(int M, int64_t K, int nw) { return q4_gemv_red_offset(M, K) + (size_t)nw * 64 * 16; }

size_t q4_gemv_lds_bytes(int M, int64_t K) { return lds_bytes_nw(M, K, GV_WAVES); }

// WPT waves share one 16-row tile, wave p taking spans p, p + WPT, ...: small
// matrices (the attention projections, the experts) then still spread over
// every SIMD.  A workgroup of NW waves covers NW / WPT tiles.
template <int WPT, int NW>
__global__ __launch_bounds__(64 * NW) void q4_gemv_kernel(const Q4GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int S = (int)(a.K / GV_SPAN), G = (int)(a.K / 64), M = a.M;
  char* xp = smem;
  char* zero = smem + (size_t)M * a.K * 2;
  float* xs = (float*)(zero + GV_ZERO);
  v4f* red = (v4f*)(smem + q4_gemv_red_offset(M, a.K));

  const int tile = blockIdx.x * (NW / WPT) + wave / WPT, part = wave % WPT;
  const bool live = tile * 16 < a.N;  // wave-uniform
  const int n_w = live && part < S ? (S - part + WPT - 1) / WPT : 0;  // spans of this wave

  const int c = lane & 15, q4 = lane >> 4;  // output column / row group, A-operand row / k quarter
  const int m = c >> 1, gs = c & 1;
  // B lanes of absent vectors, or of the other group of a span, read zeros
  const bool bval = m < M && (q4 >> 1) == gs;
  const char* bbase = bval ? xp + (((size_t)m * S) * 16 + q4) * 16 : zero + 16 * q4;
  const int bstride = bval ? 256 : 0;
  const bool xval = m < M;
  const float* xsum = xs + (xval ? m : 0) * G + gs;

  // Every span slot of the ring loads; slots past the last span load through
  // an empty resource (zeros, no memory access), so no load sits under a branch.
  const __amdgpu_buffer_rsrc_t R =
      make_rsrc(a.packed + (live ? (int64_t)tile * S * GV_REC : 0), live ? (int64_t)S * GV_REC : 0);
  const __amdgpu_buffer_rsrc_t R0 = make_rsrc(a.packed, 0);
  const uint32_t wl = 16 * lane, sl = 1024 + 16 * (2 * q4 + gs);

  constexpr int NB = 4;  // spans in flight
  v4i wbuf[NB], sbuf[NB];
#pragma unroll
  for (int i = 0; i < NB - 1; ++i) {
    const __amdgpu_buffer_rsrc_t r = i < n_w ? R : R0;
    wbuf[i] = ld128(r, wl, (part + WPT * i) * GV_REC);
    sbuf[i] = ld128(r, sl, (part + WPT * i) * GV_REC);
  }
  // (the first spans' loads above are in flight while x is staged)

  // ---- stage x: records of 8 elements in the MFMA's k order, and group sums ----
  // Thread order (m, span, gs, slab, kq & 1) puts the 8 records of one group
  // on 8 consecutive lanes.
  for (int t = tid; t < GV_ZERO / 4; t += 64 * NW) ((uint32_t*)zero)[t] = 0;
  const int nrec = M * S * 16;
  for (int t0 = 0; t0 < nrec; t0 += 64 * NW) {
    const int t = t0 + tid;
    float sum = 0.f;
    if (t < nrec) {
      const int k1 = t & 1, slab = (t >> 1) & 3, gs = (t >> 3) & 1, rest = t >> 4;
      const int span = rest % S, m = rest / S;
      const int kq = 2 * gs + k1;
      const int64_t e0 = (int64_t)span * GV_SPAN + 32 * kq + 8 * slab;
      const v4i in = *(const v4i*)(a.x + (int64_t)m * a.x_stride + e0);
      const uint32_t d0 = in[0], d1 = in[1], d2 = in[2], d3 = in[3];
      // element order of the A operand's unpack: 0, 4, 1, 5, 2, 6, 3, 7
      v4i o;
      o[0] = (int)__builtin_amdgcn_perm(d2, d0, 0x05040100u);
      o[1] = (int)__builtin_amdgcn_perm(d2, d0, 0x07060302u);
      o[2] = (int)__builtin_amdgcn_perm(d3, d1, 0x05040100u);
      o[3] = (int)__builtin_amdgcn_perm(d3, d1, 0x07060302u);
      *(v4i*)(xp + ((((size_t)m * S + span) * 4 + slab) * 4 + kq) * 16) = o;
      sum = ((bf16_lo(d0) + bf16_hi(d0)) + (bf16_lo(d1) + bf16_hi(d1))) +
            ((bf16_lo(d2) + bf16_hi(d2)) + (bf16_lo(d3) + bf16_hi(d3)));
    }
    sum = group8_sum(sum);
    if (t < nrec && (t & 7) == 0) {
      const int gs = (t >> 3) & 1, rest = t >> 4;
      xs[(rest / S) * G + 2 * (rest % S) + gs] = sum;
    }
  }
  __syncthreads();

  v4f y = {0.f, 0.f, 0.f, 0.f};
  const int n_pad = (n_w + NB - 1) / NB * NB;
  for (int i0 = 0; i0 < n_pad; i0 += NB) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int i = i0 + j, span = part + WPT * i;
      const __amdgpu_buffer_rsrc_t r = i + NB - 1 < n_w ? R : R0;
      wbuf[(j + NB - 1) % NB] = ld128(r, wl, (span + WPT * (NB - 1)) * GV_REC);
      sbuf[(j + NB - 1) % NB] = ld128(r, sl, (span + WPT * (NB - 1)) * GV_REC);
      if (i < n_w) {
        const v4i w4 = wbuf[j], sb = sbuf[j];
        const char* bp = bbase + span * bstride;
        v4f d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int slab = 0; slab < 4; ++slab) {
          const uint32_t w = (uint32_t)w4[slab];
          v4i av;
          av[0] = (int)and_or(w, 0x000f000fu, 0x43004300u);
          av[1] = (int)and_or(w >> 4, 0x000f000fu, 0x43004300u);
          av[2] = (int)and_or(w >> 8, 0x000f000fu, 0x43004300u);
          av[3] = (int)and_or(w >> 12, 0x000f000fu, 0x43004300u);
          const v4i bv = *(const v4i*)(bp + 64 * slab);
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, av), __builtin_bit_cast(v8bf, bv), d,
                                                      0, 0, 0);
        }
        const float X = xval ? xsum[2 * span] : 0.f;
        const uint32_t s01 = (uint32_t)sb[0], s23 = (uint32_t)sb[1], b01 = (uint32_t)sb[2], b23 = (uint32_t)sb[3];
        const float sc[4] = {bf16_lo(s01), bf16_hi(s01), bf16_lo(s23), bf16_hi(s23)};
        const float bi[4] = {bf16_lo(b01), bf16_hi(b01), bf16_lo(b23), bf16_hi(b23)};
#pragma unroll
        for (int r = 0; r < 4; ++r) y[r] = fmaf(fmaf(-128.f, sc[r], bi[r]), X, fmaf(sc[r], d[r], y[r]));
      }
    }
  }

  if constexpr (WPT > 1) {  // sum the partial results of the tile's waves
    red[wave * 64 + lane] = y;
    __syncthreads();
    if (part != 0) return;  // no barrier follows
#pragma unroll
    for (int p = 1; p < WPT; ++p) y += red[(wave + p) * 64 + lane];
  }
  if (!live) return;

  // the two group halves of a vector sit in lanes c, c ^ 1
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float mine = y[i];  // a copy: a bit_cast of a vector subscript reads element 0
    const int other = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, mine), 0xb1, 0xf, 0xf, false);  // quad_perm 1,0,3,2
    y[i] = mine + __builtin_bit_cast(float, other);
  }
  if (gs == 0 && m < M) {
    const int64_t r0 = (int64_t)tile * 16 + 4 * q4;
    if (a.out_dtype == DT_F32) {
      float* o = (float*)a.out + (int64_t)m * a.out_stride + r0;
      if (r0 + 3 < a.N) {
        *(v4f*)o = y;
      } else {
        for (int i = 0; i < 4; ++i)
          if (r0 + i < a.N) o[i] = y[i];
      }
    } else {
      uint16_t* o = (uint16_t*)a.out + (int64_t)m * a.out_stride + r0;
      const uint16_t h[4] = {f32_to_bf16(y[0]), f32_to_bf16(y[1]), f32_to_bf16(y[2]), f32_to_bf16(y[3])};
      if (r0 + 3 < a.N) {
        *(v2i*)o = (v2i){(int)(h[0] | ((uint32_t)h[1] << 16)), (int)(h[2] | ((uint32_t)h[3] << 16))};
      } else {
        for (int i = 0; i < 4; ++i)
          if (r0 + i < a.N) o[i] = h[i];
      }
    }
  }
}

hipError_t launch_q4_pack(const Q4PackArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)(a.K / GV_SPAN), (unsigned)((a.N + 15) / 16));
  hipLaunchKernelGGL(q4_pack_kernel, grid, dim3(64), 0, stream, a);
  return hipGetLastError();
}

template <int WPT, int NW = GV_WAVES>
hipError_t launch_q4_gemv_wpt(const Q4GemvArgs& a, int64_t tiles, hipStream_t stream) {
  constexpr int TPG = NW / WPT;  // tiles per workgroup
  const size_t lds = lds_bytes_nw(a.M, a.K, NW);
  if (lds > 65536) {
    const hipError_t e = hipFuncSetAttribute((const void*)q4_gemv_kernel<WPT, NW>,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((q4_gemv_kernel<WPT, NW>), dim3((unsigned)((tiles + TPG - 1) / TPG)), dim3(64 * NW), lds,
                     stream, a);
  return hipGetLastError();
}

hipError_t launch_q4_gemv(const Q4GemvArgs& a, hipStream_t stream) {
  const int64_t tiles = (a.N + 15) / 16, S = a.K / GV_SPAN;
  // fewest waves per tile that still give every SIMD (1024) two waves
  if (tiles >= 2048) return launch_q4_gemv_wpt<1>(a, tiles, stream);
  if (tiles >= 1024) return launch_q4_gemv_wpt<2>(a, tiles, stream);
  // Fewer tiles than CUs (o_proj 2048 x 4096, down_proj 2048 x 6144: 128
  // tiles): one tile per workgroup of 8 or 16 waves, so that each wave's
  // spans fit its ring of NB and are all in flight at once
  if (tiles < 256 && S > 4 * 4) {
    if (S <= 8 * 4 && lds_bytes_nw(a.M, a.K, 8) <= 160 * 1024) return launch_q4_gemv_wpt<8, 8>(a, tiles, stream);
    if (lds_bytes_nw(a.M, a.K, 16) <= 160 * 1024) return launch_q4_gemv_wpt<16, 16>(a, tiles, stream);
  }
  return launch_q4_gemv_wpt<4>(a, tiles, stream);
}

// ---------------------------------------------------------------------------
// Many vectors: the projections of a prefill chunk (M rows of x), over the
// same packed records.  A GEMM on bf16 MFMA 16x16x32 with the GEMV's exact
// arithmetic: codes enter as 128 + q, x as bf16, and each 64-element group's
// sums D = Σ(128 + q)x take y += s·D + (b − 128 s)·X with X = Σx over the
// group (q4_xsum_kernel, a pass of its own).  Here a k-step covers 32
// consecutive elements of one group -- lane (r, kq) takes word 4t + kq of row
// r, dword kq of record lane r + 16t -- so x enters in its own order and the
// two groups of a span accumulate apart.

// Group sums X[m][g] = Σ x[m][64g .. 64g+63] in fp32, one thread per (m, g).
__global__ __launch_bounds__(256) void q4_xsum_kernel(const Q4GemmArgs a) {
  const int64_t G = a.K / 64;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)a.M * G) return;
  const int64_t m = i / G, g = i - m * G;
  const v4i* p = (const v4i*)(a.x + m * a.x_stride + g * 64);  // 16-byte aligned rows, K % 128 == 0
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const v4i v = p[j];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t d = (uint32_t)v[e];
      s += bf16_lo(d) + bf16_hi(d);
    }
  }
  a.xsum[i] = s;
}

// Eight 4-bit codes of one word as eight bf16 values 128 + q, one and-or
// per pair: codes d and d + 4 (element order 0, 4, 1, 5, 2, 6, 3, 7, the
// order x is staged in, as the GEMV's).
__device__ __forceinline__ v8bf unpack_codes(uint32_t w) {
  v4i o;
  o[0] = (int)and_or(w, 0x000f000fu, 0x43004300u);
  o[1] = (int)and_or(w >> 4, 0x000f000fu, 0x43004300u);
  o[2] = (int)and_or(w >> 8, 0x000f000fu, 0x43004300u);
  o[3] = (int)and_or(w >> 12, 0x000f000fu, 0x43004300u);
  return __builtin_bit_cast(v8bf, o);
}

constexpr int GM_VECS = 64;    // vectors per workgroup: four 16-column tiles
constexpr int GM_ROWS = 128;   // rows per workgroup: eight 16-row tiles, two per wave
constexpr int GM_PITCH = 272;  // LDS bytes per staged vector row of a span (256 + 16: rows on distinct banks)

// Workgroup (x, y): rows 128x .. 128x+127 against vectors 64y .. 64y+63; wave w
// takes the row tiles 8x + 2w and 8x + 2w + 1.  Each span's x (64 vectors x
// 128 elements, 16 KB) and its group sums are staged once in LDS, the next
// span's fetched into registers while this one is computed (two buffers, one
// barrier per span); every x operand read from LDS feeds both row tiles.
// Lane (r, kq) of a D tile holds rows 4kq .. 4kq+3 of vector column r, whose
// scales and biases are the record's 16-byte block kq of each group.
__global__ __launch_bounds__(256) void q4_gemm_kernel(const Q4GemmArgs a) {
  __shared__ __attribute__((aligned(16))) char xl[2][GM_VECS * GM_PITCH];
  __shared__ __attribute__((aligned(16))) float xsl[2][GM_VECS * 2];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t tiles = (a.N + 15) / 16;
  const int S = (int)(a.K / GV_SPAN), G = (int)(a.K / 64);
  const int r = lane & 15, kq = lane >> 4;
  const int m0 = (int)blockIdx.y * GM_VECS;
  const int rows = min(GM_VECS, a.M - m0);  // vectors of this workgroup (>= 1)
  // the wave's two row tiles (tiles past the matrix read zeros, store nothing)
  __amdgpu_buffer_rsrc_t R[2];
  int64_t tile[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    tile[rt] = (int64_t)blockIdx.x * 8 + 2 * wave + rt;
    const bool live = tile[rt] < tiles;
    R[rt] = make_rsrc(a.packed + (live ? tile[rt] * S * GV_REC : 0), live ? (int64_t)S * GV_REC : 0);
  }
  // x and its group sums: vectors past M lie past the resources' ends and read zero
  const __amdgpu_buffer_rsrc_t RX =
      make_rsrc(a.x + (int64_t)m0 * a.x_stride, ((int64_t)(rows - 1) * a.x_stride + a.K) * 2);
  const __amdgpu_buffer_rsrc_t RS = make_rsrc(a.xsum + (int64_t)m0 * G, (int64_t)rows * G * 4);
  // staging: thread tid carries 16-byte pieces tid + 256 j (vector piece / 16,
  // piece % 16 of its 256-byte span row); threads 0-63 also the vector's two sums
  uint32_t xoff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int pc = tid + 256 * j;
    xoff[j] = (uint32_t)(((int64_t)(pc >> 4) * a.x_stride + 8 * (pc & 15)) * 2);
  }
  const uint32_t soff = (uint32_t)(tid & 63) * (uint32_t)G * 4;
  const uint32_t wl = 16 * r + 4 * kq, sl = 1024 + 32 * kq;

  v4i xr[4];
  v2i sr;
  uint32_t wr[2][4];
  v4i sbr[2][2];
  const auto fetch = [&](int sp) {
#pragma unroll
    for (int j = 0; j < 4; ++j) xr[j] = ld128<0>(RX, xoff[j] + (uint32_t)(256 * sp), 0);
    sr = ld64<0>(RS, soff + (uint32_t)(8 * sp), 0);
    const uint32_t rec = (uint32_t)sp * GV_REC;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
#pragma unroll
      for (int t = 0; t < 4; ++t) wr[rt][t] = ld32<0>(R[rt], wl + 256 * t, rec);
      sbr[rt][0] = ld128<0>(R[rt], sl, rec);
      sbr[rt][1] = ld128<0>(R[rt], sl + 16, rec);
    }
  };
  const auto stage = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // each 8-element piece in the unpack's element order 0, 4, 1, 5, 2, 6, 3, 7
      const int pc = tid + 256 * j;
      const uint32_t d0 = xr[j][0], d1 = xr[j][1], d2 = xr[j][2], d3 = xr[j][3];
      v4i o;
      o[0] = (int)__builtin_amdgcn_perm(d2, d0, 0x05040100u);
      o[1] = (int)__builtin_amdgcn_perm(d2, d0, 0x07060302u);
      o[2] = (int)__builtin_amdgcn_perm(d3, d1, 0x05040100u);
      o[3] = (int)__builtin_amdgcn_perm(d3, d1, 0x07060302u);
      *(v4i*)(xl[buf] + (pc >> 4) * GM_PITCH + 16 * (pc & 15)) = o;
    }
    if (tid < 64) *(v2i*)(xsl[buf] + 2 * tid) = sr;
  };

  v4f y[2][4];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int vt = 0; vt < 4; ++vt) y[rt][vt] = (v4f){0.f, 0.f, 0.f, 0.f};

  fetch(0);
  stage(0);
  __syncthreads();
  for (int sp = 0; sp < S; ++sp) {
    const int buf = sp & 1;
    // this span's weights (fetched with the span's x) into operands and
    // per-group coefficients, before the next span's loads reuse the registers
    v8bf av[2][4];
    float sc[2][2][4], cb[2][2][4];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
#pragma unroll
      for (int t = 0; t < 4; ++t) av[rt][t] = unpack_codes(wr[rt][t]);
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const v4i sb = sbr[rt][g];
        const uint32_t s01 = (uint32_t)sb[0], s23 = (uint32_t)sb[1], b01 = (uint32_t)sb[2], b23 = (uint32_t)sb[3];
        const float s4[4] = {bf16_lo(s01), bf16_hi(s01), bf16_lo(s23), bf16_hi(s23)};
        const float b4[4] = {bf16_lo(b01), bf16_hi(b01), bf16_lo(b23), bf16_hi(b23)};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sc[rt][g][i] = s4[i];
          cb[rt][g][i] = fmaf(-128.f, s4[i], b4[i]);
        }
      }
    }
    if (sp + 1 < S) fetch(sp + 1);
#pragma unroll
    for (int vt = 0; vt < 4; ++vt) {
      const char* xp = xl[buf] + (16 * vt + r) * GM_PITCH + 16 * kq;
      v8bf bx[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) bx[t] = *(const v8bf*)(xp + 64 * t);
      const v2f xsum = *(const v2f*)(xsl[buf] + 2 * (16 * vt + r));
      const float X0 = xsum.x, X1 = xsum.y;
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const v4f z = {0.f, 0.f, 0.f, 0.f};
        v4f d0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[rt][0], bx[0], z, 0, 0, 0);
        d0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[rt][1], bx[1], d0, 0, 0, 0);
        v4f d1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[rt][2], bx[2], z, 0, 0, 0);
        d1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[rt][3], bx[3], d1, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float acc = y[rt][vt][i];
          acc = fmaf(cb[rt][0][i], X0, fmaf(sc[rt][0][i], d0[i], acc));
          acc = fmaf(cb[rt][1][i], X1, fmaf(sc[rt][1][i], d1[i], acc));
          y[rt][vt][i] = acc;
        }
      }
    }
    if (sp + 1 < S) stage(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    if (tile[rt] >= tiles) continue;
    const int64_t n0 = tile[rt] * 16 + 4 * kq;
#pragma unroll
    for (int vt = 0; vt < 4; ++vt) {
      const int m = m0 + 16 * vt + r;
      if (m >= a.M) continue;
      const v4f v = y[rt][vt];
      if (a.out_dtype == DT_F32) {
        float* o = (float*)a.out + (int64_t)m * a.out_stride + n0;
        if (n0 + 3 < a.N) {
          *(v4f*)o = v;
        } else {
          for (int i = 0; i < 4; ++i)
            if (n0 + i < a.N) o[i] = v[i];
        }
      } else {
        uint16_t* o = (uint16_t*)a.out + (int64_t)m * a.out_stride + n0;
        const uint16_t h[4] = {f32_to_bf16(v[0]), f32_to_bf16(v[1]), f32_to_bf16(v[2]), f32_to_bf16(v[3])};
        if (n0 + 3 < a.N) {
          *(v2i*)o = (v2i){(int)(h[0] | ((uint32_t)h[1] << 16)), (int)(h[2] | ((uint32_t)h[3] << 16))};
        } else {
          for (int i = 0; i < 4; ++i)
            if (n0 + i < a.N) o[i] = h[i];
        }
      }
    }
  }
}

hipError_t launch_q4_gemm(const Q4GemmArgs& a, hipStream_t stream) {
  const int64_t sums = (int64_t)a.M * (a.K / 64);
  hipLaunchKernelGGL(q4_xsum_kernel, dim3((unsigned)((sums + 255) / 256)), dim3(256), 0, stream, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t tiles = (a.N + 15) / 16;
  hipLaunchKernelGGL(q4_gemm_kernel, dim3((unsigned)((tiles + 7) / 8), (unsigned)((a.M + GM_VECS - 1) / GM_VECS)),
                     dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace rec
