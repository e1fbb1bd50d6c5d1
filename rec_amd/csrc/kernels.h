// Argument blocks and host-side launchers of the device kernels.
#pragma once

#include "common.h"
#include "quant.h"

namespace rec {

// An additive bias on the attention scores (natural-log units, -inf drops a
// key): element (b, kv head h, group member g, query l, key t) at
//   p[b * sb + h * skv + g * sg + l * sl + t]   (key stride 1, strides 0 where
// a dimension broadcasts), the reference's mask array after its broadcasting
// (engine/src/rec_mlx/model.py:122-128).  extent: elements readable from p
// (reads past a row's T keys fall on masked positions or past the extent,
// where the buffer loads read zero).
struct BiasArgs {
  const float* p;  // null: no bias
  int64_t sb, skv, sg, sl;
  int64_t extent;
};

struct AppendArgs {
  RowSrc k, v;
  void* kq;
  uint16_t* ks;
  uint16_t* kz;
  void* vq;
  uint16_t* vs;
  uint16_t* vz;
  int B, Hkv, L;
  int64_t offset, cap;
  int64_t v_units;  // per (b, h): L rows, or byte pairs for uint4 V
};

struct DecodeArgs {
  const void* q;
  int q_dtype;
  int64_t q_sb, q_sh;  // element strides of q (batch, head); dims contiguous
  const void* kq;
  const uint16_t* ks;
  const uint16_t* kz;
  const void* vq;
  const uint16_t* vs;
  const uint16_t* vz;
  const float* sinks;  // [Hq] or null
  void* out;           // [B][Hq][128], out_dtype
  int out_dtype;       // DT_F32, DT_BF16 or DT_F16
  float* ws_acc;       // [B*Hkv][S][8][128]
  float* ws_stat;      // [B*Hkv][S][8][2]
  int64_t k_sb, k_sh, v_sb, v_sh;  // bf16 K/V (B, Hkv, T, 128) element strides (token stride 128)
  RowSrc knew, vnew;   // fused single-token append (knew.p null: none)
  float q_mul;         // softmax scale * log2(e)
  int B, Hq, Hkv, G;
  int64_t T, cap;
  int S;     // number of splits
  int span;         // tokens per regular split (multiple of 32)
  int t_split_end;  // end of the regular splits; a fused append adds one split [t_split_end, T)
  int64_t new_pos;  // bf16 fused write: the new token's position (T - 1, or its ring slot)
  BiasArgs bias;    // additive score bias (a mask array), or none
};

// P·V takes the V-scaled probabilities P' = p·s as an fp16 operand.  Rounded
// once, each carries a relative error up to 2^-11; for a query row that sees
// n keys the output error is about 2^-12·|v|·sqrt(Σ w_t²) (w the softmax
// weights), which stays inside 2e-3 once the weights spread over a few
// hundred keys, but not for a row that sees a handful of keys with large,
// cancelling values.  So below this many visible keys the kernels carry P'
// as a high and a low fp16 part (exact to ~2^-22): in the decode for the
// 4-bit and affine V formats (int8 V always takes both parts, at almost no
// cost), and in the prefill, where the low part costs a second P·V MFMA.
constexpr int64_t EXACT_PV_BELOW = 8192;

struct PrefillArgs {
  const void* q;
  int q_dtype;                 // DT_BF16 (bf16 MFMA) or DT_F16 (fp16 MFMA)
  int64_t q_sb, q_sh, q_st;    // element strides of q (batch, head, position)
  int q_vec;                   // q rows 16-byte aligned, strides multiples of 8 elements: vector loads
  int k_fmt, v_fmt;            // 8, 4, FMT_A8 / FMT_A4, or FMT_BF (bf16 tensors, strides below)
  const void* kq;              // K codes (cache layout) or bf16 K
  const uint16_t* ks;          // scales (affine: [scale, bias])
  const uint16_t* kz;          // uint4 zero-points
  const void* vq;
  const uint16_t* vs;
  const uint16_t* vz;
  const float* sinks;          // [Hq] or null
  void* out;                   // [B][Hq][L][128], out_dtype
  int out_dtype;               // DT_F32, DT_BF16 or DT_F16
  float q_mul;                 // softmax scale * log2(e)
  int B, Hq, Hkv, G, L;
  int64_t T, cap;              // cached tokens including the L new ones; capacity
  int causal;
  int window;                  // > 0: query at position p sees keys (p - window, p] only
  int kv_bf16;                 // k_fmt == v_fmt == FMT_BF
  int64_t k_sb, k_sh, v_sb, v_sh;
  // split-K over the keys (S > 1): workgroup (qb, s) scans keys
  // [split_lo + s * split_len, + split_len) of its query block's range and
  // writes an unnormalised partial; prefill_merge_kernel combines them
  int S, nqb, block_rows;      // splits, query blocks of block_rows (query, head) rows
  int64_t split_lo, split_len;
  BiasArgs bias;               // additive score bias (a mask array), or none
  float* ws_acc;               // [B*Hkv][S][nqb][block_rows][128]
  float* ws_stat;              // [B*Hkv][S][nqb][block_rows] x (max, sum)
};

// Prefill split plan: how many key splits a launch uses and where they lie.
constexpr int PREFILL_MAX_SPLITS = 64;
// (query, head) rows per prefill workgroup: a KV head's rows are numbered
// query * G + head, and workgroup qb takes rows [R qb, R qb + R), R =
// PREFILL_BLOCK_ROWS (an automatic plan for a windowed launch may take 128
// or 64)
constexpr int PREFILL_BLOCK_ROWS = 256;
struct PrefillPlan {
  int S, nqb, block_rows;
  int64_t split_lo, split_len;
};
// requested <= 0: automatic (splits only when the query blocks x KV heads x
// batch grid is too small to fill the chip); else at most `requested`
PrefillPlan prefill_plan(const PrefillArgs& a, int requested);
// workspace bytes for S splits of head_rows (= nqb x block_rows) rows per KV
// head (0 when S == 1); accumulators then statistics
size_t prefill_ws_bytes(int B, int Hkv, int64_t head_rows, int S);

// Cache rows [0, T) dequantized to bf16 (B, Hkv, T, 128) tensors.
struct DequantArgs {
  const void* kq;
  const uint16_t* ks;
  const uint16_t* kz;
  const void* vq;
  const uint16_t* vs;
  const uint16_t* vz;
  int B, Hkv;
  int64_t T, cap;
  uint16_t* k_out;
  uint16_t* v_out;
};

// int4 group-64 GEMV: repack of an MLX affine matrix, then y = x Wᵀ.
struct Q4PackArgs {
  const uint32_t* w;        // [N][K/8] MLX words
  const uint16_t* scales;   // [N][K/64] bf16
  const uint16_t* biases;   // [N][K/64] bf16
  int64_t N, K;
  uint8_t* packed;          // [ceil(N/16)][K/128][1152 B]
};

struct Q4GemvArgs {
  const uint8_t* packed;
  int64_t N, K;
  const uint16_t* x;        // [M][x_stride] bf16
  int64_t x_stride;
  int M;                    // 1..8 vectors
  void* out;                // [M][out_stride] bf16 or fp32
  int out_dtype;            // DT_BF16 or DT_F32
  int64_t out_stride;
};

// Many vectors (a prefill chunk's projections): the same packed matrix as a
// GEMM.  xsum: [M][K/64] fp32 group sums of x (workspace, written first).
struct Q4GemmArgs {
  const uint8_t* packed;
  int64_t N, K;
  const uint16_t* x;        // [M][x_stride] bf16
  int64_t x_stride;
  int M;
  float* xsum;              // [M][K/64]
  void* out;                // [M][out_stride] bf16 or fp32
  int out_dtype;            // DT_BF16 or DT_F32
  int64_t out_stride;
};

constexpr int DECODE_MAX_SPLITS = 256;
constexpr int Q4_MAX_M = 8;

hipError_t launch_append(int kb, int vb, const AppendArgs& a, hipStream_t stream);
hipError_t launch_fill_zero(uint32_t* p, int64_t words, hipStream_t stream);
hipError_t launch_stream_read(const void* p, int64_t n16, int workgroups, uint32_t* out, hipStream_t stream);
hipError_t launch_decode_partial(int kb, int vb, const DecodeArgs& a, hipStream_t stream);
hipError_t launch_decode_merge(const DecodeArgs& a, hipStream_t stream);
hipError_t launch_prefill(const PrefillArgs& a, hipStream_t stream);  // both kernels when a.S > 1
// A few queries over a quantized cache, no window and no mask array: the
// streaming kernel of prefill_few.hip, whose partials share the tiled
// kernel's workspace layout and merge.  Up to PREFILL_FEW_ROWS (query, head)
// rows per KV head over any cache, and up to PREFILL_BLOCK_ROWS over
// 16,384-131,071 keys, in row groups of one workgroup each
// (prefill_few_groups of them)
constexpr int PREFILL_FEW_ROWS = 64;
bool prefill_few_fits(const PrefillArgs& a);
int prefill_few_groups(const PrefillArgs& a);
hipError_t launch_prefill_few(const PrefillArgs& a, hipStream_t stream);
hipError_t launch_decode_bf16(const DecodeArgs& a, hipStream_t stream);
hipError_t launch_dequant(int kb, int vb, const DequantArgs& a, hipStream_t stream);
hipError_t launch_q4_pack(const Q4PackArgs& a, hipStream_t stream);
hipError_t launch_q4_gemv(const Q4GemvArgs& a, hipStream_t stream);
size_t q4_gemv_lds_bytes(int M, int64_t K);
hipError_t launch_q4_gemm(const Q4GemmArgs& a, hipStream_t stream);
hipError_t launch_ring_join_bf16(const AppendArgs& a, void* rk, void* rv, int64_t rk_sb, int64_t rk_sh,
                                 int64_t rv_sb, int64_t rv_sh, int64_t head, int64_t n, int64_t keep_from, bool place,
                                 void* ok, void* ov, hipStream_t stream);
hipError_t launch_write_bf16(const AppendArgs& a, int64_t k_sb, int64_t k_sh, int64_t v_sb, int64_t v_sh,
                             hipStream_t stream);

}  // namespace rec
