// Quantize-on-append of L new K/V rows into the cache (gfx950).
//
// Restates MixedQuantizedKVCache.update_and_fetch's write step
// (engine/src/rec_mlx/model.py:76-81): rows [0, L) of the new keys/values are
// quantized and stored at cache positions [offset, offset + L).  One wavefront
// per row (4-bit V: per byte pair of positions), four per workgroup.  Formats:
// int8 / uint4 (this library's), and MLX-style affine 8-bit K with 4-bit V.
#include "kernels.h"

namespace rec {


// Workgroups per launch of the row kernels, at most: they stride over the
// rows, so any row count stays inside the dispatch's 32-bit thread count.
constexpr int64_t ROW_GRID_MAX = 1 << 20;

__host__ __device__ inline unsigned row_grid(int64_t rows) {
  const int64_t wgs = (rows + 3) / 4;
  return (unsigned)(wgs < ROW_GRID_MAX ? (wgs > 0 ? wgs : 1) : ROW_GRID_MAX);
}

// blockIdx.y: 0 = K, 1 = V
template <int KB, int VB>
__global__ __launch_bounds__(256) void append_kernel(const AppendArgs a) {
  const int lane = threadIdx.x & 63;
  const int kind = blockIdx.y;
  const int64_t per_bh = kind == 0 ? a.L : a.v_units;
  const int64_t total = (int64_t)a.B * a.Hkv * per_bh;
  for (int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); unit < total; unit += (int64_t)gridDim.x * 4) {
    const int64_t bh = unit / per_bh, u = unit % per_bh;
    const int b = (int)(bh / a.Hkv), h = (int)(bh % a.Hkv);
    if (kind == 0) {
      append_row<KB>(a.k, b, h, (int)u, 0, a.kq, a.ks, a.kz, bh, a.cap, a.offset + u, lane);
    } else if constexpr (VB == 8) {
      append_row<8>(a.v, b, h, (int)u, 1, a.vq, a.vs, nullptr, bh, a.cap, a.offset + u, lane);
    } else {
      const int64_t pos_even = ((a.offset >> 1) + u) * 2;
      const bool has_even = pos_even >= a.offset && pos_even < a.offset + a.L;
      const bool has_odd = pos_even + 1 >= a.offset && pos_even + 1 < a.offset + a.L;
      append_v4_pair<is_a4(VB), meta_f16(VB)>(a.v, b, h, (int)(pos_even - a.offset), has_even, has_odd,
                                              (uint8_t*)a.vq, a.vs, a.vz, bh, a.cap, pos_even, lane);
    }
  }
}

// Dequantize cache rows [0, T) to bf16 (B, Hkv, T, 128) tensors: the
// reference's prefill branch dequantizes the cache to the query dtype before
// its attention (engine/src/rec_mlx/model.py:194-195).  One wavefront per row,
// lane l owns dims 2l, 2l+1; x̂ is formed in float32 exactly as the CPU
// restatement does (int8 q·s, uint4 (q - z)·s, affine q·s + b), then rounded
// to bf16.  blockIdx.y: 0 = K, 1 = V.
template <int BITS>
__device__ __forceinline__ void dequant_pair(const void* codes, const uint16_t* scales, const uint16_t* zeros,
                                             bool is_v, int64_t bh, int64_t cap, int64_t t, int lane, float& x0,
                                             float& x1) {
  const int d = 2 * lane;
  if constexpr (BITS == 8) {
    const int8_t* c = (const int8_t*)codes;
    const int q0 = is_v ? c[v8_off(bh, cap, t, d)] : c[k8_off(bh, cap, t, d)];
    const int q1 = is_v ? c[v8_off(bh, cap, t, d + 1)] : c[k8_off(bh, cap, t, d + 1)];
    const float s = half_bits_to_float(scales[s8_off(bh, cap, t)]);
    x0 = (float)q0 * s;
    x1 = (float)q1 * s;
  } else if constexpr (BITS == 4) {
    const uint8_t* c = (const uint8_t*)codes;
    int q0, q1;
    if (is_v) {
      const int p = block_pos((int)(t & 31));
      const uint8_t b0 = c[v4_off(bh, cap, t, d)], b1 = c[v4_off(bh, cap, t, d + 1)];
      q0 = (p & 1) ? b0 >> 4 : b0 & 15;
      q1 = (p & 1) ? b1 >> 4 : b1 & 15;
    } else {
      const uint8_t b = c[k4_off(bh, cap, t, d)];
      q0 = b & 15;
      q1 = b >> 4;
    }
    const int g = d >> 5;
    const float s = half_bits_to_float(scales[s4_off(bh, cap, t, g)]);
    const float z = half_bits_to_float(zeros[s4_off(bh, cap, t, g)]);
    x0 = ((float)q0 - z) * s;
    x1 = ((float)q1 - z) * s;
  } else {  // affine: 8-bit keys (uint8 in the int8 K layout), 4-bit values (uint4 in the int4 V layout)
    const uint8_t* c = (const uint8_t*)codes;
    int q0, q1;
    if constexpr (is_a8(BITS)) {
      q0 = c[k8_off(bh, cap, t, d)];
      q1 = c[k8_off(bh, cap, t, d + 1)];
    } else {
      const int p = block_pos((int)(t & 31));
      const uint8_t b0 = c[v4_off(bh, cap, t, d)], b1 = c[v4_off(bh, cap, t, d + 1)];
      q0 = (p & 1) ? b0 >> 4 : b0 & 15;
      q1 = (p & 1) ? b1 >> 4 : b1 & 15;
    }
    const int g = d >> 6;
    const float s = meta_bits<meta_f16(BITS)>(scales[sa_off(bh, cap, t, 0, g)]);
    const float b = meta_bits<meta_f16(BITS)>(scales[sa_off(bh, cap, t, 1, g)]);
    x0 = (float)q0 * s + b;
    x1 = (float)q1 * s + b;
  }
}

template <int KB, int VB>
__global__ __launch_bounds__(256) void dequant_kernel(const DequantArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t total = (int64_t)a.B * a.Hkv * a.T;
  const bool is_v = blockIdx.y == 1;
  for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < total; row += (int64_t)gridDim.x * 4) {
    const int64_t bh = row / a.T, t = row % a.T;
    float x0, x1;
    if (!is_v) dequant_pair<KB>(a.kq, a.ks, a.kz, false, bh, a.cap, t, lane, x0, x1);
    else dequant_pair<VB>(a.vq, a.vs, a.vz, true, bh, a.cap, t, lane, x0, x1);
    uint16_t* o = (is_v ? a.v_out : a.k_out) + row * HEAD_DIM + 2 * lane;
    *(uint32_t*)o = (uint32_t)float_to_bf16_bits(x0) | ((uint32_t)float_to_bf16_bits(x1) << 16);
  }
}

hipError_t launch_dequant(int kb, int vb, const DequantArgs& a, hipStream_t stream) {
  const int64_t rows = (int64_t)a.B * a.Hkv * a.T;
  const dim3 grid(row_grid(rows), 2), block(256);
  if (kb == 8 && vb == 8) hipLaunchKernelGGL((dequant_kernel<8, 8>), grid, block, 0, stream, a);
  else if (kb == 8 && vb == 4) hipLaunchKernelGGL((dequant_kernel<8, 4>), grid, block, 0, stream, a);
  else if (kb == 4 && vb == 8) hipLaunchKernelGGL((dequant_kernel<4, 8>), grid, block, 0, stream, a);
  else if (kb == FMT_A8 && vb == FMT_A4) hipLaunchKernelGGL((dequant_kernel<FMT_A8, FMT_A4>), grid, block, 0, stream, a);
  else if (kb == FMT_A8H && vb == FMT_A4H)
    hipLaunchKernelGGL((dequant_kernel<FMT_A8H, FMT_A4H>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((dequant_kernel<4, 4>), grid, block, 0, stream, a);
  return hipGetLastError();
}

// Zero a word range (graph-safe replacement for hipMemsetAsync).
__global__ void fill_zero_kernel(uint32_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

hipError_t launch_append(int kb, int vb, const AppendArgs& a, hipStream_t stream) {
  const int64_t rows = (int64_t)a.B * a.Hkv * (a.L > a.v_units ? a.L : a.v_units);
  const dim3 grid(row_grid(rows), 2), block(256);
  if (kb == 8 && vb == 8) hipLaunchKernelGGL((append_kernel<8, 8>), grid, block, 0, stream, a);
  else if (kb == 8 && vb == 4) hipLaunchKernelGGL((append_kernel<8, 4>), grid, block, 0, stream, a);
  else if (kb == 4 && vb == 8) hipLaunchKernelGGL((append_kernel<4, 8>), grid, block, 0, stream, a);
  else if (kb == FMT_A8 && vb == FMT_A4) hipLaunchKernelGGL((append_kernel<FMT_A8, FMT_A4>), grid, block, 0, stream, a);
  else if (kb == FMT_A8H && vb == FMT_A4H)
    hipLaunchKernelGGL((append_kernel<FMT_A8H, FMT_A4H>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((append_kernel<4, 4>), grid, block, 0, stream, a);
  return hipGetLastError();
}

// A plain streaming read of n16 16-byte chunks: consecutive lanes read
// consecutive chunks (1 KB per wavefront and load), four loads in flight per
// lane, grid-stride.  The XOR of everything read is stored only when it hits a
// fixed value, so the loads stay live without a store per lane.  The read floor
// the decode kernels are measured against.
__global__ __launch_bounds__(256) void stream_read_kernel(const v4i* p, int64_t n16, uint32_t* out) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  v4i acc = {0, 0, 0, 0};
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const v4i a = __builtin_nontemporal_load(p + i), b = __builtin_nontemporal_load(p + i + stride);
    const v4i c = __builtin_nontemporal_load(p + i + 2 * stride), d = __builtin_nontemporal_load(p + i + 3 * stride);
    acc ^= a ^ b ^ c ^ d;
  }
  for (; i < n16; i += stride) acc ^= __builtin_nontemporal_load(p + i);
  const uint32_t x = (uint32_t)(acc[0] ^ acc[1] ^ acc[2] ^ acc[3]);
  if (x == 0x9e3779b9u) out[blockIdx.x] = x;
}

hipError_t launch_stream_read(const void* p, int64_t n16, int workgroups, uint32_t* out, hipStream_t stream) {
  hipLaunchKernelGGL(stream_read_kernel, dim3(workgroups), dim3(256), 0, stream, (const v4i*)p, n16, out);
  return hipGetLastError();
}

hipError_t launch_fill_zero(uint32_t* p, int64_t words, hipStream_t stream) {
  if (words <= 0) return hipSuccess;
  const int64_t wgs = (words + 255) / 256;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)(wgs < ROW_GRID_MAX ? wgs : ROW_GRID_MAX)), dim3(256), 0, stream,
                     p, words);
  return hipGetLastError();
}

}  // namespace rec
