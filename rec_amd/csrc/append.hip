// Quantize-on-append of L new K/V rows into the cache (gfx950).
//
// Restates MixedQuantizedKVCache.update_and_fetch's write step
// (engine/src/rec_mlx/model.py:76-81): rows [0, L) of the new keys/values are
// quantized and stored at cache positions [offset, offset + L).  One wavefront
// per row (4-bit V: per byte pair of positions), four per workgroup.  Formats:
// int8 / uint4 (this library's), and MLX-style affine 8-bit K with 4-bit V.
#include "kernels.h"

namespace rec {


// blockIdx.y: 0 = K, 1 = V
template <int KB, int VB>
__global__ __launch_bounds__(256) void append_kernel(const AppendArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int kind = blockIdx.y;
  const int64_t per_bh = kind == 0 ? a.L : a.v_units;
  if (unit >= (int64_t)a.B * a.Hkv * per_bh) return;
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
    append_v4_pair<VB == FMT_A4>(a.v, b, h, (int)(pos_even - a.offset), has_even, has_odd, (uint8_t*)a.vq, a.vs,
                                 a.vz, bh, a.cap, pos_even, lane);
  }
}

// Zero a word range (graph-safe replacement for hipMemsetAsync).
__global__ void fill_zero_kernel(uint32_t* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

hipError_t launch_append(int kb, int vb, const AppendArgs& a, hipStream_t stream) {
  const int64_t rows = (int64_t)a.B * a.Hkv * (a.L > a.v_units ? a.L : a.v_units);
  const dim3 grid((unsigned)((rows + 3) / 4), 2), block(256);
  if (kb == 8 && vb == 8) hipLaunchKernelGGL((append_kernel<8, 8>), grid, block, 0, stream, a);
  else if (kb == 8 && vb == 4) hipLaunchKernelGGL((append_kernel<8, 4>), grid, block, 0, stream, a);
  else if (kb == 4 && vb == 8) hipLaunchKernelGGL((append_kernel<4, 8>), grid, block, 0, stream, a);
  else if (kb == FMT_A8 && vb == FMT_A4) hipLaunchKernelGGL((append_kernel<FMT_A8, FMT_A4>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((append_kernel<4, 4>), grid, block, 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_fill_zero(uint32_t* p, int64_t words, hipStream_t stream) {
  if (words <= 0) return hipSuccess;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, stream, p, words);
  return hipGetLastError();
}

}  // namespace rec
