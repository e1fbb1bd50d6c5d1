// C ABI of the library: argument validation, workspace layout and launches.
// Declarations and the reference interface each entry point replaces are in
// include/rec_amd.h.
#include <stdarg.h>
#include <stdio.h>

#include <cmath>
#include <mutex>
#include <vector>

#include "../../include/rec_amd.h"
#include "kernels.h"

using namespace rec;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = 0;
  return REC_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Rows of p can be read with vector loads: 16-byte aligned base, strides that
// keep every row start 16-byte aligned for 4-byte elements (8 for 2-byte).
int vec_rows(const void* p, int64_t s0, int64_t s1, int64_t s2) {
  return aligned16(p) && s0 % 4 == 0 && s1 % 4 == 0 && s2 % 4 == 0;
}

int launched(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(REC_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

size_t round256(size_t x) { return (x + 255) & ~(size_t)255; }

// Prefill query rows (2-byte elements) that the kernel can read with 16-byte
// loads: aligned base, strides that keep every 8-element run aligned.
int query_rows_vec(const void* q, int64_t sb, int64_t sh, int64_t st) {
  return aligned16(q) && sb % 8 == 0 && sh % 8 == 0 && st % 8 == 0;
}

struct WorkspaceLayout {
  size_t stat, acc, total;
};

// Split partials: stats (m, l) then accumulators, per (b, h, split, head-in-group).
WorkspaceLayout ws_layout(int B, int Hkv, int splits) {
  WorkspaceLayout w;
  const size_t bh = (size_t)B * Hkv;
  w.stat = 0;
  w.acc = round256(bh * splits * 8 * 2 * sizeof(float));
  w.total = w.acc + bh * splits * 8 * HEAD_DIM * sizeof(float);
  return w;
}

int check_bits(int bits, const char* name) {
  if (bits != 8 && bits != 4) return fail(REC_EINVAL, "%s must be 8 or 4, got %d", name, bits);
  return REC_OK;
}

// (k_bits, v_bits) -> kernel formats: this library's 8 / 4 in any mix, or
// the MLX-style affine pair REC_AFFINE8 keys with REC_AFFINE4 values (bf16
// scales and biases), or REC_AFFINE8_F16 with REC_AFFINE4_F16 (fp16).
int resolve_formats(int k_bits, int v_bits, int* kf, int* vf) {
  const auto affine = [](int c) {
    return c == REC_AFFINE8 || c == REC_AFFINE4 || c == REC_AFFINE8_F16 || c == REC_AFFINE4_F16;
  };
  if (affine(k_bits) || affine(v_bits)) {
    if (k_bits == REC_AFFINE8 && v_bits == REC_AFFINE4) {
      *kf = FMT_A8;
      *vf = FMT_A4;
    } else if (k_bits == REC_AFFINE8_F16 && v_bits == REC_AFFINE4_F16) {
      *kf = FMT_A8H;
      *vf = FMT_A4H;
    } else {
      return fail(REC_EUNSUPPORTED,
                  "the affine formats are REC_AFFINE8 keys with REC_AFFINE4 values, or REC_AFFINE8_F16 with "
                  "REC_AFFINE4_F16 (got %#x, %#x)",
                  k_bits, v_bits);
    }
    return REC_OK;
  }
  int e;
  if ((e = check_bits(k_bits, "k_bits")) || (e = check_bits(v_bits, "v_bits"))) return e;
  *kf = k_bits;
  *vf = v_bits;
  return REC_OK;
}

int check_cache(int bits, const void* codes, const void* scales, const void* zeros, const char* name) {
  if (!codes || !scales) return fail(REC_EINVAL, "%s codes/scales pointer is null", name);
  if (bits == 4 && !zeros) return fail(REC_EINVAL, "%s zero-points are required for 4-bit", name);
  if (!aligned16(codes) || !aligned16(scales) || (bits == 4 && !aligned16(zeros)))
    return fail(REC_EALIGN, "%s cache buffers must be 16-byte aligned", name);
  return REC_OK;
}

int check_dtype(int dt, const char* name) {
  if (dt != REC_F16 && dt != REC_BF16 && dt != REC_F32) return fail(REC_EINVAL, "%s dtype %d is not f16/bf16/f32", name, dt);
  return REC_OK;
}

// A score bias (mask array): 16-byte aligned, strides non-negative multiples
// of 4 elements (the kernels read four keys per 16-byte load), extent below
// 2^29 elements (byte offsets fit a 32-bit buffer offset).  null: no bias.
int make_bias(const float* p, int64_t sb, int64_t skv, int64_t sg, int64_t sl, int64_t extent, BiasArgs* out) {
  *out = BiasArgs{};
  if (!p) return REC_OK;
  if (!aligned16(p)) return fail(REC_EALIGN, "bias must be 16-byte aligned");
  if (sb < 0 || skv < 0 || sg < 0 || sl < 0 || sb % 4 || skv % 4 || sg % 4 || sl % 4)
    return fail(REC_EALIGN, "bias strides must be non-negative multiples of 4 elements");
  if (extent < 1 || extent >= ((int64_t)1 << 29))
    return fail(REC_EUNSUPPORTED, "bias extent of %lld elements (1 .. 2^29 - 1 supported)", (long long)extent);
  *out = BiasArgs{p, sb, skv, sg, sl, extent};
  return REC_OK;
}

// Splits actually launched for a request.  Regular splits cover
// [0, t_split_end) in spans of whole 32-token chunks; with a fused append the
// newest token's chunk [t_split_end, T) is one more split of its own, so the
// append's latency is not added to a full-size split.
constexpr int CHUNK = BLOCK_T;
void effective_splits(int64_t T, int req, bool fused, int* S, int* span, int* t_split_end) {
  const int64_t R = fused ? ((T - 1) / CHUNK) * CHUNK : T;
  int S_reg = 0, sp = CHUNK;
  if (R > 0) {
    const int64_t chunks = (R + CHUNK - 1) / CHUNK;
    int64_t s = req - (fused ? 1 : 0);
    if (s < 1) s = 1;
    if (s > chunks) s = chunks;
    const int64_t span_chunks = (chunks + s - 1) / s;
    sp = (int)(span_chunks * CHUNK);
    S_reg = (int)((chunks + span_chunks - 1) / span_chunks);
  }
  *S = S_reg + (fused ? 1 : 0);
  *span = sp;
  *t_split_end = (int)R;
}

int decode_common(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int k_bits, const void* kq,
                  const uint16_t* ks, const uint16_t* kz, int v_bits, const void* vq, const uint16_t* vs,
                  const uint16_t* vz, const float* sinks, float scale, int B, int Hq, int Hkv, int D, int64_t T,
                  int64_t cap, int splits, void* ws, size_t ws_bytes, int out_dtype, void* out,
                  const RowSrc* knew, const RowSrc* vnew, int phases, void* stream, const BiasArgs* bias = nullptr) {
  int e;
  if ((e = resolve_formats(k_bits, v_bits, &k_bits, &v_bits))) return e;
  if ((e = check_dtype(q_dtype, "query"))) return e;
  if ((e = check_dtype(out_dtype, "output"))) return e;
  if (D != HEAD_DIM) return fail(REC_EUNSUPPORTED, "head_dim %d is not supported (128 only)", D);
  if (B < 1 || Hkv < 1 || Hq < 1) return fail(REC_EINVAL, "B, Hq and Hkv must be positive");
  if (Hq % Hkv != 0) return fail(REC_EINVAL, "Hq (%d) must be a multiple of Hkv (%d)", Hq, Hkv);
  if (Hq / Hkv > 8) return fail(REC_EUNSUPPORTED, "GQA ratio %d exceeds 8", Hq / Hkv);
  if (T < 1) return fail(REC_EINVAL, "decode needs at least one cached token (T=%lld)", (long long)T);
  if (cap % BLOCK_T != 0) return fail(REC_EINVAL, "capacity %lld is not a multiple of 32", (long long)cap);
  if (T > cap) return fail(REC_ECAPACITY, "T=%lld exceeds the cache capacity %lld", (long long)T, (long long)cap);
  if (cap > ((int64_t)1 << 24)) return fail(REC_EUNSUPPORTED, "capacity above 16M tokens per head");
  if (!q || !out) return fail(REC_EINVAL, "query/output pointer is null");
  if (!aligned16(out)) return fail(REC_EALIGN, "output must be 16-byte aligned");
  if (!vec_rows(q, q_sb, q_sh, 0))
    return fail(REC_EALIGN, "query rows must start 16-byte aligned (strides multiples of 4 elements)");
  if ((e = check_cache(k_bits, kq, ks, kz, "key")) || (e = check_cache(v_bits, vq, vs, vz, "value"))) return e;
  if (!std::isfinite(scale)) return fail(REC_EINVAL, "scale must be finite");
  if (splits <= 0) splits = rec_decode_default_splits(B, Hkv, T);
  if (splits > DECODE_MAX_SPLITS) splits = DECODE_MAX_SPLITS;
  int S, span, t_split_end;
  effective_splits(T, splits, knew != nullptr, &S, &span, &t_split_end);
  const WorkspaceLayout w = ws_layout(B, Hkv, S);
  if ((phases != 0 && !ws) || ws_bytes < w.total)
    return fail(REC_EWORKSPACE, "workspace of %zu bytes is too small (%zu needed for %d splits)", ws_bytes, w.total, S);
  if (phases == 0) return ok();  // validation only
  if (!aligned16(ws)) return fail(REC_EALIGN, "workspace must be 16-byte aligned");
  DecodeArgs a{};
  a.q = q;
  a.q_dtype = q_dtype;
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.kq = kq;
  a.ks = ks;
  a.kz = kz;
  a.vq = vq;
  a.vs = vs;
  a.vz = vz;
  a.sinks = sinks;
  a.out = out;
  a.out_dtype = out_dtype;
  if (bias) a.bias = *bias;
  a.ws_stat = (float*)((char*)ws + w.stat);
  a.ws_acc = (float*)((char*)ws + w.acc);
  if (knew) {
    a.knew = *knew;
    a.vnew = *vnew;
  }
  a.q_mul = scale * LOG2E;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.G = Hq / Hkv;
  a.T = T;
  a.cap = cap;
  a.S = S;
  a.span = span;
  a.t_split_end = t_split_end;
  if (phases & 1) {
    const int e1 = launched(launch_decode_partial(k_bits, v_bits, a, (hipStream_t)stream), "decode launch");
    if (e1 != REC_OK) return e1;
  }
  if (phases & 2) return launched(launch_decode_merge(a, (hipStream_t)stream), "merge launch");
  return ok();
}

// ---- allocation-free decode: split partials in a static device array ----
}  // namespace

constexpr size_t SCRATCH_BYTES = (size_t)8 << 20;
static __device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];

namespace {
// `scratch` is a device-side array of every GPU the library runs on (each
// holds its own copy until the process ends).  Host code never uses its name
// as an address: the first call on a device resolves that device's copy with
// hipGetSymbolAddress and keeps the pointer, which the kernels then take as
// their workspace.

constexpr int SCRATCH_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[SCRATCH_MAX_DEVICES] = {};

// This device's scratch pointer (resolved on its first use), or null with the
// error set.
void* device_scratch(int* rc) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= SCRATCH_MAX_DEVICES) {
    *rc = fail(REC_ELAUNCH, "no current device for the static scratch: %s", hipGetErrorString(e));
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      *rc = fail(REC_ELAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" {

const char* rec_version(void) { return "rec_amd 0.1.0 gfx950"; }

const char* rec_last_error(void) { return g_err; }

int rec_kv_append(const void* k_new, const void* v_new, int in_dtype, int64_t k_sb, int64_t k_sh, int64_t k_st,
                  int64_t v_sb, int64_t v_sh, int64_t v_st, int k_bits, void* k_codes, uint16_t* k_scales,
                  uint16_t* k_zeros, int v_bits, void* v_codes, uint16_t* v_scales, uint16_t* v_zeros, int B,
                  int Hkv, int L, int D, int64_t offset, int64_t capacity, void* stream) {
  int e;
  if ((e = resolve_formats(k_bits, v_bits, &k_bits, &v_bits))) return e;
  if ((e = check_dtype(in_dtype, "input"))) return e;
  if (D != HEAD_DIM) return fail(REC_EUNSUPPORTED, "head_dim %d is not supported (128 only)", D);
  if (B < 1 || Hkv < 1 || L < 0) return fail(REC_EINVAL, "bad shape B=%d Hkv=%d L=%d", B, Hkv, L);
  if (offset < 0) return fail(REC_EINVAL, "negative offset");
  if (capacity % BLOCK_T != 0) return fail(REC_EINVAL, "capacity %lld is not a multiple of 32", (long long)capacity);
  if (offset + L > capacity)
    return fail(REC_ECAPACITY, "appending %d tokens at %lld exceeds the capacity %lld", L, (long long)offset,
                (long long)capacity);
  if (L == 0) return ok();
  if (!k_new || !v_new) return fail(REC_EINVAL, "new keys/values pointer is null");
  if ((e = check_cache(k_bits, k_codes, k_scales, k_zeros, "key")) ||
      (e = check_cache(v_bits, v_codes, v_scales, v_zeros, "value")))
    return e;
  AppendArgs a{};
  a.k = RowSrc{k_new, in_dtype, k_sb, k_sh, k_st, vec_rows(k_new, k_sb, k_sh, k_st)};
  a.v = RowSrc{v_new, in_dtype, v_sb, v_sh, v_st, vec_rows(v_new, v_sb, v_sh, v_st)};
  a.kq = k_codes;
  a.ks = k_scales;
  a.kz = k_zeros;
  a.vq = v_codes;
  a.vs = v_scales;
  a.vz = v_zeros;
  a.B = B;
  a.Hkv = Hkv;
  a.L = L;
  a.offset = offset;
  a.cap = capacity;
  a.v_units = v_bits == 4 || is_a4(v_bits) ? ((offset + L - 1) >> 1) - (offset >> 1) + 1 : L;
  return launched(launch_append(k_bits, v_bits, a, (hipStream_t)stream), "append launch");
}

int rec_decode_default_splits(int B, int Hkv, int64_t T) {
  // One workgroup per CU (256 CUs) across all (b, h) pairs: measured best at
  // 32K-252K tokens (two per CU, or uneven counts, leave some CUs a second
  // round); at least one 32-token chunk per split.
  const int64_t target = 256;
  const int64_t bh = (int64_t)(B < 1 ? 1 : B) * (Hkv < 1 ? 1 : Hkv);
  int64_t s = (target + bh - 1) / bh;
  const int64_t chunks = (T + CHUNK - 1) / CHUNK;
  if (s > chunks) s = chunks;
  if (s > DECODE_MAX_SPLITS) s = DECODE_MAX_SPLITS;
  return (int)(s < 1 ? 1 : s);
}

size_t rec_decode_workspace_bytes(int B, int Hkv, int splits) {
  if (splits <= 0 || splits > DECODE_MAX_SPLITS) splits = DECODE_MAX_SPLITS;
  // a fused append adds the newest token's split to max(splits - 1, 1)
  // regular ones (effective_splits), so a request for one split launches two
  if (splits < 2) splits = 2;
  return ws_layout(B, Hkv, splits).total;
}

int rec_workspace_init(void* workspace, size_t workspace_bytes, void* stream) {
  if (!workspace) return fail(REC_EWORKSPACE, "workspace is null");
  if (!aligned16(workspace)) return fail(REC_EALIGN, "workspace must be 16-byte aligned");
  return launched(launch_fill_zero((uint32_t*)workspace, (int64_t)(workspace_bytes / 4), (hipStream_t)stream),
                  "workspace init");
}

int rec_decode_attn(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int k_bits, const void* k_codes,
                    const uint16_t* k_scales, const uint16_t* k_zeros, int v_bits, const void* v_codes,
                    const uint16_t* v_scales, const uint16_t* v_zeros, const float* sinks, float scale,
                    const float* bias, int64_t bias_sb, int64_t bias_skv, int64_t bias_sg, int64_t bias_extent,
                    int B, int Hq, int Hkv, int D, int64_t T, int64_t capacity, int splits, void* workspace,
                    size_t workspace_bytes, int out_dtype, void* out, void* stream) {
  BiasArgs bz;
  if (int e = make_bias(bias, bias_sb, bias_skv, bias_sg, 0, bias_extent, &bz)) return e;
  return decode_common(q, q_dtype, q_sb, q_sh, k_bits, k_codes, k_scales, k_zeros, v_bits, v_codes, v_scales, v_zeros,
                       sinks, scale, B, Hq, Hkv, D, T, capacity, splits, workspace, workspace_bytes, out_dtype, out,
                       nullptr, nullptr, 3, stream, &bz);
}

static int append_attn(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, const void* k_new, const void* v_new,
                       int new_dtype, int64_t k_sb, int64_t k_sh, int64_t v_sb, int64_t v_sh, int k_bits,
                       void* k_codes, uint16_t* k_scales, uint16_t* k_zeros, int v_bits, void* v_codes,
                       uint16_t* v_scales, uint16_t* v_zeros, const float* sinks, float scale, int B, int Hq, int Hkv,
                       int D, int64_t T, int64_t capacity, int splits, void* workspace, size_t workspace_bytes,
                       int out_dtype, void* out, int phases, void* stream) {
  const bool append = k_new != nullptr || v_new != nullptr;
  if (append) {
    int e;
    if ((e = check_dtype(new_dtype, "new keys/values"))) return e;
    if (!k_new || !v_new) return fail(REC_EINVAL, "new keys and values must both be given");
  }
  const RowSrc kn{k_new, new_dtype, k_sb, k_sh, 0, vec_rows(k_new, k_sb, k_sh, 0)},
      vn{v_new, new_dtype, v_sb, v_sh, 0, vec_rows(v_new, v_sb, v_sh, 0)};
  return decode_common(q, q_dtype, q_sb, q_sh, k_bits, k_codes, k_scales, k_zeros, v_bits, v_codes, v_scales, v_zeros,
                       sinks, scale, B, Hq, Hkv, D, T, capacity, splits, workspace, workspace_bytes, out_dtype, out,
                       append ? &kn : nullptr, append ? &vn : nullptr, phases, stream);
}

int rec_decode_append_attn(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, const void* k_new,
                           const void* v_new, int new_dtype, int64_t k_sb, int64_t k_sh, int64_t v_sb, int64_t v_sh,
                           int k_bits, void* k_codes, uint16_t* k_scales, uint16_t* k_zeros, int v_bits,
                           void* v_codes, uint16_t* v_scales, uint16_t* v_zeros, const float* sinks, float scale,
                           int B, int Hq, int Hkv, int D, int64_t T, int64_t capacity, int splits, void* workspace,
                           size_t workspace_bytes, int out_dtype, void* out, void* stream) {
  if (!k_new || !v_new) return fail(REC_EINVAL, "new keys/values pointer is null");
  return append_attn(q, q_dtype, q_sb, q_sh, k_new, v_new, new_dtype, k_sb, k_sh, v_sb, v_sh, k_bits, k_codes,
                     k_scales, k_zeros, v_bits, v_codes, v_scales, v_zeros, sinks, scale, B, Hq, Hkv, D, T, capacity,
                     splits, workspace, workspace_bytes, out_dtype, out, 3, stream);
}

size_t rec_decode_scratch_bytes(void) { return SCRATCH_BYTES; }

int rec_decode_append_attn_noalloc(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, const void* k_new,
                                   const void* v_new, int new_dtype, int64_t k_sb, int64_t k_sh, int64_t v_sb,
                                   int64_t v_sh, int k_bits, void* k_codes, uint16_t* k_scales, uint16_t* k_zeros,
                                   int v_bits, void* v_codes, uint16_t* v_scales, uint16_t* v_zeros,
                                   const float* sinks, float scale, int B, int Hq, int Hkv, int D, int64_t T,
                                   int64_t capacity, int splits, int out_dtype, void* out, void* stream) {
  if (!k_new || !v_new) return fail(REC_EINVAL, "new keys/values pointer is null");
  // validate everything, the plan's partials against the scratch size included, before touching the device
  int e = append_attn(q, q_dtype, q_sb, q_sh, k_new, v_new, new_dtype, k_sb, k_sh, v_sb, v_sh, k_bits, k_codes,
                      k_scales, k_zeros, v_bits, v_codes, v_scales, v_zeros, sinks, scale, B, Hq, Hkv, D, T, capacity,
                      splits, nullptr, SCRATCH_BYTES, out_dtype, out, 0, stream);
  if (e == REC_EWORKSPACE) {
    char why[sizeof(g_err)];
    snprintf(why, sizeof(why), "%s", g_err);
    return fail(REC_EWORKSPACE,
                "the split partials exceed the library's %zu-byte static scratch (%s); request fewer splits or "
                "use rec_decode_append_attn with a workspace",
                SCRATCH_BYTES, why);
  }
  if (e != REC_OK) return e;
  void* ws = device_scratch(&e);
  if (!ws) return e;
  return append_attn(q, q_dtype, q_sb, q_sh, k_new, v_new, new_dtype, k_sb, k_sh, v_sb, v_sh, k_bits, k_codes,
                     k_scales, k_zeros, v_bits, v_codes, v_scales, v_zeros, sinks, scale, B, Hq, Hkv, D, T, capacity,
                     splits, ws, SCRATCH_BYTES, out_dtype, out, 3, stream);
}

int rec_decode_partial(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, const void* k_new, const void* v_new,
                       int new_dtype, int64_t k_sb, int64_t k_sh, int64_t v_sb, int64_t v_sh, int k_bits,
                       void* k_codes, uint16_t* k_scales, uint16_t* k_zeros, int v_bits, void* v_codes,
                       uint16_t* v_scales, uint16_t* v_zeros, const float* sinks, float scale, int B, int Hq, int Hkv,
                       int D, int64_t T, int64_t capacity, int splits, void* workspace, size_t workspace_bytes,
                       int out_dtype, void* out, void* stream) {
  return append_attn(q, q_dtype, q_sb, q_sh, k_new, v_new, new_dtype, k_sb, k_sh, v_sb, v_sh, k_bits, k_codes,
                     k_scales, k_zeros, v_bits, v_codes, v_scales, v_zeros, sinks, scale, B, Hq, Hkv, D, T, capacity,
                     splits, workspace, workspace_bytes, out_dtype, out, 1, stream);
}

int rec_decode_merge(const float* sinks, int B, int Hq, int Hkv, int64_t T, int splits, int appended, void* workspace,
                     size_t workspace_bytes, int out_dtype, void* out, void* stream) {
  if (B < 1 || Hkv < 1 || Hq < 1 || Hq % Hkv != 0 || Hq / Hkv > 8 || T < 1)
    return fail(REC_EINVAL, "bad shape B=%d Hq=%d Hkv=%d T=%lld", B, Hq, Hkv, (long long)T);
  if (int e = check_dtype(out_dtype, "output")) return e;
  if (!out || !aligned16(out)) return fail(REC_EALIGN, "output must be a 16-byte aligned buffer");
  if (splits <= 0) splits = rec_decode_default_splits(B, Hkv, T);
  if (splits > DECODE_MAX_SPLITS) splits = DECODE_MAX_SPLITS;
  int S, span, t_split_end;
  effective_splits(T, splits, appended != 0, &S, &span, &t_split_end);
  const WorkspaceLayout w = ws_layout(B, Hkv, S);
  if (!workspace || workspace_bytes < w.total) return fail(REC_EWORKSPACE, "workspace too small");
  DecodeArgs a{};
  a.sinks = sinks;
  a.out = out;
  a.out_dtype = out_dtype;
  a.ws_stat = (float*)((char*)workspace + w.stat);
  a.ws_acc = (float*)((char*)workspace + w.acc);
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.G = Hq / Hkv;
  a.T = T;
  a.S = S;
  return launched(launch_decode_merge(a, (hipStream_t)stream), "merge launch");
}

// Key splits of a prefill launch: the plan for `splits` (<= 0: automatic),
// which needs a workspace when it splits; an automatic plan without one runs
// unsplit, an explicit split count without one is an error.
static int plan_prefill_splits(PrefillArgs& a, int splits, void* workspace, size_t workspace_bytes) {
  if (splits > PREFILL_MAX_SPLITS) return fail(REC_EINVAL, "splits %d exceeds %d", splits, PREFILL_MAX_SPLITS);
  PrefillPlan p = prefill_plan(a, splits);
  size_t need = prefill_ws_bytes(a.B, a.Hkv, (int64_t)p.nqb * p.block_rows, p.S);
  if (need > 0 && (!workspace || workspace_bytes < need)) {
    if (splits > 1)
      return fail(REC_EWORKSPACE, "workspace of %zu bytes is smaller than the %zu that %d splits need",
                  workspace ? workspace_bytes : (size_t)0, need, splits);
    p = prefill_plan(a, 1);
    need = 0;
  }
  if (need > 0 && !aligned16(workspace)) return fail(REC_EALIGN, "workspace must be 16-byte aligned");
  a.S = p.S;
  a.nqb = p.nqb;
  a.block_rows = p.block_rows;
  a.split_lo = p.split_lo;
  a.split_len = p.split_len;
  if (p.S > 1) {
    const size_t rows = (size_t)a.B * a.Hkv * p.S * p.nqb * p.block_rows;
    a.ws_acc = (float*)workspace;
    a.ws_stat = (float*)((char*)workspace + rows * HEAD_DIM * 4);
  }
  return REC_OK;
}

size_t rec_prefill_workspace_bytes(int B, int Hq, int Hkv, int L, int splits) {
  if (B < 1 || Hkv < 1 || L < 1 || Hq < Hkv || Hq % Hkv != 0) return 0;
  const int nqb = (int)(((int64_t)L * (Hq / Hkv) + PREFILL_BLOCK_ROWS - 1) / PREFILL_BLOCK_ROWS);
  int S = splits;
  if (S <= 0) {  // the automatic plan's most (prefill_plan): two splits from half the chip to three quarters
    const int64_t nwg = (int64_t)nqb * Hkv * B;
    S = nwg >= 192 ? 1 : nwg >= 128 ? 2 : (int)std::min<int64_t>(PREFILL_MAX_SPLITS, (256 + nwg - 1) / nwg);
  }
  // (blocks of 256 rows: the most any plan needs; smaller blocks take fewer splits)
  return prefill_ws_bytes(B, Hkv, (int64_t)nqb * PREFILL_BLOCK_ROWS, std::min(S, PREFILL_MAX_SPLITS));
}

int rec_prefill_attn(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st, int k_bits,
                     const void* k_codes, const uint16_t* k_scales, const uint16_t* k_zeros, int v_bits,
                     const void* v_codes, const uint16_t* v_scales, const uint16_t* v_zeros, const float* sinks,
                     float scale, int causal, int window, const float* bias, int64_t bias_sb, int64_t bias_skv,
                     int64_t bias_sg, int64_t bias_sl, int64_t bias_extent, int B, int Hq, int Hkv, int D, int L, int64_t T,
                     int64_t capacity, int splits, void* workspace, size_t workspace_bytes, int out_dtype, void* out,
                     void* stream) {
  int e;
  int kf, vf;
  if ((e = resolve_formats(k_bits, v_bits, &kf, &vf))) return e;
  if ((e = check_dtype(out_dtype, "output"))) return e;
  if (q_dtype != REC_BF16 && q_dtype != REC_F16)
    return fail(REC_EUNSUPPORTED, "prefill queries must be bf16 or f16 (the matrix-core input type)");
  if (D != HEAD_DIM) return fail(REC_EUNSUPPORTED, "head_dim %d is not supported (128 only)", D);
  if (B < 1 || Hkv < 1 || Hq < 1 || L < 1) return fail(REC_EINVAL, "bad shape B=%d Hq=%d Hkv=%d L=%d", B, Hq, Hkv, L);
  if (Hq % Hkv != 0) return fail(REC_EINVAL, "Hq (%d) must be a multiple of Hkv (%d)", Hq, Hkv);
  if (Hq / Hkv > 8) return fail(REC_EUNSUPPORTED, "GQA ratio %d exceeds 8", Hq / Hkv);
  if (T < L) return fail(REC_EINVAL, "T=%lld is smaller than L=%d (the new tokens are cached first)", (long long)T, L);
  if (capacity % BLOCK_T != 0) return fail(REC_EINVAL, "capacity %lld is not a multiple of 32", (long long)capacity);
  if (T > capacity) return fail(REC_ECAPACITY, "T=%lld exceeds the cache capacity %lld", (long long)T, (long long)capacity);
  if (capacity > ((int64_t)1 << 24)) return fail(REC_EUNSUPPORTED, "capacity above 16M tokens per head");
  if (window < 0) return fail(REC_EINVAL, "negative window");
  if (!q || !out) return fail(REC_EINVAL, "query/output pointer is null");
  if (!aligned16(out)) return fail(REC_EALIGN, "output must be 16-byte aligned");
  if ((e = check_cache(kf, k_codes, k_scales, k_zeros, "key")) || (e = check_cache(vf, v_codes, v_scales, v_zeros, "value")))
    return e;
  BiasArgs bz;
  if ((e = make_bias(bias, bias_sb, bias_skv, bias_sg, bias_sl, bias_extent, &bz))) return e;
  if (bias && (causal || window))
    return fail(REC_EINVAL, "a bias (mask array) carries the whole mask: causal and window must be 0 with it");
  if (!std::isfinite(scale)) return fail(REC_EINVAL, "scale must be finite");
  PrefillArgs a{};
  a.q = q;
  a.q_dtype = q_dtype;
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.q_st = q_st;
  a.q_vec = query_rows_vec(q, q_sb, q_sh, q_st);
  a.k_fmt = kf;
  a.v_fmt = vf;
  a.kq = k_codes;
  a.ks = k_scales;
  a.kz = k_zeros;
  a.vq = v_codes;
  a.vs = v_scales;
  a.vz = v_zeros;
  a.sinks = sinks;
  a.out = out;
  a.out_dtype = out_dtype;
  a.bias = bz;
  a.q_mul = scale * LOG2E;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.G = Hq / Hkv;
  a.L = L;
  a.T = T;
  a.cap = capacity;
  a.causal = causal != 0;
  a.window = window;
  if ((e = plan_prefill_splits(a, splits, workspace, workspace_bytes))) return e;
  return launched(launch_prefill(a, (hipStream_t)stream), "prefill launch");
}

int rec_kv_dequant_bf16(int k_bits, const void* k_codes, const uint16_t* k_scales, const uint16_t* k_zeros, int v_bits,
                        const void* v_codes, const uint16_t* v_scales, const uint16_t* v_zeros, int B, int Hkv,
                        int64_t T, int64_t capacity, void* k_out, void* v_out, void* stream) {
  int e, kf, vf;
  if ((e = resolve_formats(k_bits, v_bits, &kf, &vf))) return e;
  if (B < 1 || Hkv < 1 || T < 0) return fail(REC_EINVAL, "bad shape B=%d Hkv=%d T=%lld", B, Hkv, (long long)T);
  if (capacity % BLOCK_T != 0) return fail(REC_EINVAL, "capacity %lld is not a multiple of 32", (long long)capacity);
  if (T > capacity) return fail(REC_ECAPACITY, "T=%lld exceeds the cache capacity %lld", (long long)T, (long long)capacity);
  if ((e = check_cache(kf, k_codes, k_scales, k_zeros, "key")) || (e = check_cache(vf, v_codes, v_scales, v_zeros, "value")))
    return e;
  if (!k_out || !v_out) return fail(REC_EINVAL, "output pointer is null");
  if (!aligned16(k_out) || !aligned16(v_out)) return fail(REC_EALIGN, "outputs must be 16-byte aligned");
  if (T == 0) return ok();
  DequantArgs a{};
  a.kq = k_codes;
  a.ks = k_scales;
  a.kz = k_zeros;
  a.vq = v_codes;
  a.vs = v_scales;
  a.vz = v_zeros;
  a.B = B;
  a.Hkv = Hkv;
  a.T = T;
  a.cap = capacity;
  a.k_out = (uint16_t*)k_out;
  a.v_out = (uint16_t*)v_out;
  return launched(launch_dequant(kf, vf, a, (hipStream_t)stream), "dequant launch");
}

int rec_prefill_bf16(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st, const void* k, int64_t k_sb,
                     int64_t k_sh, const void* v, int64_t v_sb, int64_t v_sh, const float* sinks, float scale,
                     int causal, int window, const float* bias, int64_t bias_sb, int64_t bias_skv, int64_t bias_sg,
                     int64_t bias_sl, int64_t bias_extent, int B, int Hq, int Hkv, int D, int L, int64_t T, int splits,
                     void* workspace, size_t workspace_bytes, int out_dtype, void* out, void* stream) {
  if (q_dtype != REC_BF16 && q_dtype != REC_F16)
    return fail(REC_EUNSUPPORTED, "prefill queries must be bf16 or f16 (the matrix-core input type)");
  if (int e = check_dtype(out_dtype, "output")) return e;
  if (D != HEAD_DIM) return fail(REC_EUNSUPPORTED, "head_dim %d is not supported (128 only)", D);
  if (B < 1 || Hkv < 1 || Hq < 1 || L < 1) return fail(REC_EINVAL, "bad shape B=%d Hq=%d Hkv=%d L=%d", B, Hq, Hkv, L);
  if (Hq % Hkv != 0) return fail(REC_EINVAL, "Hq (%d) must be a multiple of Hkv (%d)", Hq, Hkv);
  if (Hq / Hkv > 8) return fail(REC_EUNSUPPORTED, "GQA ratio %d exceeds 8", Hq / Hkv);
  if (T < L) return fail(REC_EINVAL, "T=%lld is smaller than L=%d (the new tokens are cached first)", (long long)T, L);
  if (T > ((int64_t)1 << 24)) return fail(REC_EUNSUPPORTED, "T above 16M tokens");
  if (window < 0) return fail(REC_EINVAL, "negative window");
  if (!q || !out || !k || !v) return fail(REC_EINVAL, "null pointer");
  if (!aligned16(out) || !aligned16(k) || !aligned16(v)) return fail(REC_EALIGN, "K, V and output must be 16-byte aligned");
  if (k_sb % 8 || k_sh % 8 || v_sb % 8 || v_sh % 8)
    return fail(REC_EALIGN, "K/V batch and head strides must be multiples of 8 elements");
  if (!std::isfinite(scale)) return fail(REC_EINVAL, "scale must be finite");
  BiasArgs bz;
  if (int e = make_bias(bias, bias_sb, bias_skv, bias_sg, bias_sl, bias_extent, &bz)) return e;
  if (bias && (causal || window))
    return fail(REC_EINVAL, "a bias (mask array) carries the whole mask: causal and window must be 0 with it");
  PrefillArgs a{};
  a.q = q;
  a.q_dtype = q_dtype;
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.q_st = q_st;
  a.q_vec = query_rows_vec(q, q_sb, q_sh, q_st);
  a.k_fmt = a.v_fmt = FMT_BF;
  a.kq = k;
  a.vq = v;
  a.k_sb = k_sb;
  a.k_sh = k_sh;
  a.v_sb = v_sb;
  a.v_sh = v_sh;
  a.kv_bf16 = 1;
  a.sinks = sinks;
  a.out = out;
  a.out_dtype = out_dtype;
  a.bias = bz;
  a.q_mul = scale * LOG2E;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.G = Hq / Hkv;
  a.L = L;
  a.T = T;
  a.cap = T;
  a.causal = causal != 0;
  a.window = window;
  if (int e = plan_prefill_splits(a, splits, workspace, workspace_bytes)) return e;
  return launched(launch_prefill(a, (hipStream_t)stream), "prefill launch");
}

int rec_kv_write_bf16(const void* k_new, const void* v_new, int in_dtype, int64_t k_sb, int64_t k_sh, int64_t k_st,
                      int64_t v_sb, int64_t v_sh, int64_t v_st, void* k, int64_t kc_sb, int64_t kc_sh, void* v,
                      int64_t vc_sb, int64_t vc_sh, int B, int Hkv, int L, int D, int64_t offset, int64_t capacity,
                      void* stream) {
  int e;
  if ((e = check_dtype(in_dtype, "input"))) return e;
  if (D != HEAD_DIM) return fail(REC_EUNSUPPORTED, "head_dim %d is not supported (128 only)", D);
  if (B < 1 || Hkv < 1 || L < 0) return fail(REC_EINVAL, "bad shape B=%d Hkv=%d L=%d", B, Hkv, L);
  if (offset < 0) return fail(REC_EINVAL, "negative offset");
  if (offset + L > capacity)
    return fail(REC_ECAPACITY, "writing %d tokens at %lld exceeds the capacity %lld", L, (long long)offset,
                (long long)capacity);
  if (L == 0) return ok();
  if (!k_new || !v_new || !k || !v) return fail(REC_EINVAL, "null key/value pointer");
  if (!vec_rows(k, kc_sb, kc_sh, 0) || !vec_rows(v, vc_sb, vc_sh, 0))
    return fail(REC_EALIGN, "bf16 K/V storage must be 16-byte aligned with strides that are multiples of 8 elements");
  if (kc_sb % 8 || kc_sh % 8 || vc_sb % 8 || vc_sh % 8)
    return fail(REC_EALIGN, "bf16 K/V storage strides must be multiples of 8 elements");
  AppendArgs a{};
  a.k = RowSrc{k_new, in_dtype, k_sb, k_sh, k_st, vec_rows(k_new, k_sb, k_sh, k_st)};
  a.v = RowSrc{v_new, in_dtype, v_sb, v_sh, v_st, vec_rows(v_new, v_sb, v_sh, v_st)};
  a.kq = k;
  a.vq = v;
  a.B = B;
  a.Hkv = Hkv;
  a.L = L;
  a.offset = offset;
  a.cap = capacity;
  return launched(launch_write_bf16(a, kc_sb, kc_sh, vc_sb, vc_sh, (hipStream_t)stream), "bf16 write launch");
}

int rec_ring_join_bf16(void* k_ring, void* v_ring, int64_t rk_sb, int64_t rk_sh, int64_t rv_sb,
                       int64_t rv_sh, int64_t capacity, int64_t head, int64_t n_held, int64_t offset, int place,
                       const void* k_new,
                       const void* v_new, int in_dtype, int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t v_sb,
                       int64_t v_sh, int64_t v_st, void* k_out, void* v_out, int B, int Hkv, int L, int D,
                       void* stream) {
  int e;
  if ((e = check_dtype(in_dtype, "input"))) return e;
  if (D != HEAD_DIM) return fail(REC_EUNSUPPORTED, "head_dim %d is not supported (128 only)", D);
  if (B < 1 || Hkv < 1 || L < 0) return fail(REC_EINVAL, "bad shape B=%d Hkv=%d L=%d", B, Hkv, L);
  if (capacity < 1 || n_held < 0 || n_held > capacity || head < 0 || head >= capacity)
    return fail(REC_EINVAL, "ring of capacity %lld cannot hold %lld tokens from slot %lld", (long long)capacity,
                (long long)n_held, (long long)head);
  if (offset < 0) return fail(REC_EINVAL, "negative offset");
  if (n_held + L == 0) return ok();
  if (!k_out || !v_out || ((n_held > 0 || place) && (!k_ring || !v_ring)) || (L > 0 && (!k_new || !v_new)))
    return fail(REC_EINVAL, "null key/value pointer");
  if ((reinterpret_cast<uintptr_t>(k_out) | reinterpret_cast<uintptr_t>(v_out)) & 3)
    return fail(REC_EALIGN, "joined K/V must be 4-byte aligned");
  if ((n_held > 0 || place) && (((reinterpret_cast<uintptr_t>(k_ring) | reinterpret_cast<uintptr_t>(v_ring)) & 3) ||
                     ((rk_sb | rk_sh | rv_sb | rv_sh) & 1)))
    return fail(REC_EALIGN, "ring K/V must be 4-byte aligned with even strides");
  AppendArgs a{};
  a.k = RowSrc{k_new, in_dtype, k_sb, k_sh, k_st, L > 0 && vec_rows(k_new, k_sb, k_sh, k_st)};
  a.v = RowSrc{v_new, in_dtype, v_sb, v_sh, v_st, L > 0 && vec_rows(v_new, v_sb, v_sh, v_st)};
  a.B = B;
  a.Hkv = Hkv;
  a.L = L;
  a.cap = capacity;
  a.offset = offset;
  const int64_t keep_from = L - std::min<int64_t>(L, capacity);
  return launched(launch_ring_join_bf16(a, k_ring, v_ring, rk_sb, rk_sh, rv_sb, rv_sh, head, n_held, keep_from,
                                        place != 0, k_out, v_out, (hipStream_t)stream),
                  "ring join launch");
}

static int decode_bf16(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, const void* k_new, const void* v_new,
                       int new_dtype, int64_t kn_sb, int64_t kn_sh, int64_t vn_sb, int64_t vn_sh, void* k,
                       int64_t k_sb, int64_t k_sh, void* v, int64_t v_sb, int64_t v_sh, const float* sinks,
                       float scale, int B, int Hq, int Hkv, int D, int64_t T, int64_t capacity, int splits,
                       void* workspace, size_t workspace_bytes, int out_dtype, void* out, void* stream,
                       int64_t new_pos, const BiasArgs& bias) {
  int e;
  if ((e = check_dtype(q_dtype, "query"))) return e;
  if ((e = check_dtype(out_dtype, "output"))) return e;
  if (D != HEAD_DIM) return fail(REC_EUNSUPPORTED, "head_dim %d is not supported (128 only)", D);
  if (B < 1 || Hkv < 1 || Hq < 1) return fail(REC_EINVAL, "B, Hq and Hkv must be positive");
  if (Hq % Hkv != 0) return fail(REC_EINVAL, "Hq (%d) must be a multiple of Hkv (%d)", Hq, Hkv);
  if (Hq / Hkv > 8) return fail(REC_EUNSUPPORTED, "GQA ratio %d exceeds 8", Hq / Hkv);
  if (T < 1) return fail(REC_EINVAL, "decode needs at least one cached token (T=%lld)", (long long)T);
  if (T > capacity) return fail(REC_ECAPACITY, "T=%lld exceeds the cache capacity %lld", (long long)T, (long long)capacity);
  if (T > ((int64_t)1 << 23)) return fail(REC_EUNSUPPORTED, "more than 8M tokens per head");
  if (!q || !out || !k || !v) return fail(REC_EINVAL, "null query/output/key/value pointer");
  if (!aligned16(out)) return fail(REC_EALIGN, "output must be 16-byte aligned");
  if (!vec_rows(q, q_sb, q_sh, 0))
    return fail(REC_EALIGN, "query rows must start 16-byte aligned (strides multiples of 4 elements)");
  if (!aligned16(k) || !aligned16(v) || k_sb % 8 || k_sh % 8 || v_sb % 8 || v_sh % 8)
    return fail(REC_EALIGN, "bf16 K/V must be 16-byte aligned with strides that are multiples of 8 elements");
  if (!std::isfinite(scale)) return fail(REC_EINVAL, "scale must be finite");
  const bool append = k_new != nullptr || v_new != nullptr;
  if (append) {
    if ((e = check_dtype(new_dtype, "new keys/values"))) return e;
    if (!k_new || !v_new) return fail(REC_EINVAL, "new keys and values must both be given");
  }
  if (splits <= 0) splits = rec_decode_default_splits(B, Hkv, T);
  if (splits > DECODE_MAX_SPLITS) splits = DECODE_MAX_SPLITS;
  int S, span, t_split_end;
  effective_splits(T, splits, append, &S, &span, &t_split_end);
  const WorkspaceLayout w = ws_layout(B, Hkv, S);
  if (S > 1 && (!workspace || workspace_bytes < w.total))
    return fail(REC_EWORKSPACE, "workspace of %zu bytes is too small (%zu needed for %d splits)", workspace_bytes,
                w.total, S);
  if (!aligned16(workspace)) return fail(REC_EALIGN, "workspace must be 16-byte aligned");
  DecodeArgs a{};
  a.q = q;
  a.q_dtype = q_dtype;
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.kq = k;
  a.vq = v;
  a.k_sb = k_sb;
  a.k_sh = k_sh;
  a.v_sb = v_sb;
  a.v_sh = v_sh;
  a.sinks = sinks;
  a.out = out;
  a.out_dtype = out_dtype;
  a.bias = bias;
  a.ws_stat = (float*)((char*)workspace + w.stat);
  a.ws_acc = (float*)((char*)workspace + w.acc);
  if (append) {
    a.knew = RowSrc{k_new, new_dtype, kn_sb, kn_sh, 0, vec_rows(k_new, kn_sb, kn_sh, 0)};
    a.vnew = RowSrc{v_new, new_dtype, vn_sb, vn_sh, 0, vec_rows(v_new, vn_sb, vn_sh, 0)};
  }
  a.q_mul = scale * LOG2E;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.G = Hq / Hkv;
  a.T = T;
  a.cap = capacity;
  a.S = S;
  a.span = span;
  a.t_split_end = t_split_end;
  a.new_pos = new_pos;
  const int e1 = launched(launch_decode_bf16(a, (hipStream_t)stream), "bf16 decode launch");
  if (e1 != REC_OK) return e1;
  return launched(launch_decode_merge(a, (hipStream_t)stream), "merge launch");
}

int rec_decode_bf16(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, const void* k_new, const void* v_new,
                    int new_dtype, int64_t kn_sb, int64_t kn_sh, int64_t vn_sb, int64_t vn_sh, void* k, int64_t k_sb,
                    int64_t k_sh, void* v, int64_t v_sb, int64_t v_sh, const float* sinks, float scale,
                    const float* bias, int64_t bias_sb, int64_t bias_skv, int64_t bias_sg, int64_t bias_extent, int B,
                    int Hq, int Hkv, int D, int64_t T, int64_t capacity, int splits, void* workspace,
                    size_t workspace_bytes, int out_dtype, void* out, void* stream) {
  BiasArgs bz;
  if (int e = make_bias(bias, bias_sb, bias_skv, bias_sg, 0, bias_extent, &bz)) return e;
  return decode_bf16(q, q_dtype, q_sb, q_sh, k_new, v_new, new_dtype, kn_sb, kn_sh, vn_sb, vn_sh, k, k_sb, k_sh, v,
                     v_sb, v_sh, sinks, scale, B, Hq, Hkv, D, T, capacity, splits, workspace, workspace_bytes,
                     out_dtype, out, stream, T - 1, bz);
}

int rec_decode_bf16_ring(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, const void* k_new,
                         const void* v_new, int new_dtype, int64_t kn_sb, int64_t kn_sh, int64_t vn_sb, int64_t vn_sh,
                         void* k, int64_t k_sb, int64_t k_sh, void* v, int64_t v_sb, int64_t v_sh,
                         const float* sinks, float scale, int B, int Hq, int Hkv, int D, int64_t T,
                         int64_t capacity, int64_t slot, int splits, void* workspace, size_t workspace_bytes,
                         int out_dtype, void* out, void* stream) {
  if (!k_new || !v_new) return fail(REC_EINVAL, "a ring decode step writes its new token: k_new and v_new are required");
  if (slot < 0 || slot >= T) return fail(REC_EINVAL, "slot %lld outside the %lld occupied slots", (long long)slot, (long long)T);
  return decode_bf16(q, q_dtype, q_sb, q_sh, k_new, v_new, new_dtype, kn_sb, kn_sh, vn_sb, vn_sh, k, k_sb, k_sh, v,
                     v_sb, v_sh, sinks, scale, B, Hq, Hkv, D, T, capacity, splits, workspace, workspace_bytes,
                     out_dtype, out, stream, slot, BiasArgs{});
}

size_t rec_q4_packed_bytes(int64_t N, int64_t K) {
  if (N < 1 || K < 128 || K % 128 != 0) return 0;
  return (size_t)((N + 15) / 16) * (size_t)(K / 128) * 1152;
}

int rec_q4_pack(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, int64_t N, int64_t K,
                void* packed, size_t packed_bytes, void* stream) {
  const size_t need = rec_q4_packed_bytes(N, K);
  if (need == 0) return fail(REC_EINVAL, "q4 matrix must have N >= 1 and K a positive multiple of 128 (N=%lld K=%lld)",
                             (long long)N, (long long)K);
  if (!w || !scales || !biases || !packed) return fail(REC_EINVAL, "q4 pack: null pointer");
  if (!aligned16(w) || !aligned16(packed)) return fail(REC_EALIGN, "q4 pack: w and packed must be 16-byte aligned");
  if (packed_bytes < need) return fail(REC_EWORKSPACE, "q4 pack: packed buffer has %zu bytes, needs %zu", packed_bytes, need);
  if ((N + 15) / 16 > 65535) return fail(REC_EUNSUPPORTED, "q4 pack: N=%lld exceeds 1048560 rows", (long long)N);
  Q4PackArgs a;
  a.w = w;
  a.scales = scales;
  a.biases = biases;
  a.N = N;
  a.K = K;
  a.packed = (uint8_t*)packed;
  return launched(launch_q4_pack(a, (hipStream_t)stream), "q4 pack launch");
}

int rec_q4_gemv(const void* packed, int64_t N, int64_t K, const uint16_t* x, int64_t x_stride, int M, void* out,
                int out_dtype, int64_t out_stride, void* stream) {
  if (rec_q4_packed_bytes(N, K) == 0)
    return fail(REC_EINVAL, "q4 matrix must have N >= 1 and K a positive multiple of 128 (N=%lld K=%lld)",
                (long long)N, (long long)K);
  if (M < 1 || M > Q4_MAX_M) return fail(REC_EINVAL, "q4 gemv: M=%d vectors, 1..%d supported", M, Q4_MAX_M);
  if (!packed || !x || !out) return fail(REC_EINVAL, "q4 gemv: null pointer");
  if (out_dtype != REC_BF16 && out_dtype != REC_F32) return fail(REC_EINVAL, "q4 gemv: out dtype must be bf16 or f32");
  if (M > 1 && (x_stride < K || out_stride < N))
    return fail(REC_EINVAL, "q4 gemv: row strides (%lld, %lld) shorter than rows (%lld, %lld)", (long long)x_stride,
                (long long)out_stride, (long long)K, (long long)N);
  if (!aligned16(packed) || !aligned16(x) || (M > 1 && x_stride % 8 != 0))
    return fail(REC_EALIGN, "q4 gemv: packed and x must be 16-byte aligned, x_stride a multiple of 8");
  if (q4_gemv_lds_bytes(M, K) > 160 * 1024)
    return fail(REC_EUNSUPPORTED, "q4 gemv: M=%d vectors of K=%lld exceed the LDS staging", M, (long long)K);
  Q4GemvArgs a;
  a.packed = (const uint8_t*)packed;
  a.N = N;
  a.K = K;
  a.x = x;
  a.x_stride = x_stride;
  a.M = M;
  a.out = out;
  a.out_dtype = out_dtype == REC_F32 ? DT_F32 : DT_BF16;
  a.out_stride = out_stride;
  return launched(launch_q4_gemv(a, (hipStream_t)stream), "q4 gemv launch");
}

size_t rec_q4_gemm_workspace_bytes(int M, int64_t K) {
  if (M < 1 || K < 128 || K % 128 != 0) return 0;
  return ((size_t)M * (size_t)(K / 64) * 4 + 15) & ~(size_t)15;
}

int rec_q4_gemm(const void* packed, int64_t N, int64_t K, const uint16_t* x, int64_t x_stride, int M, void* out,
                int out_dtype, int64_t out_stride, void* workspace, size_t workspace_bytes, void* stream) {
  if (rec_q4_packed_bytes(N, K) == 0)
    return fail(REC_EINVAL, "q4 matrix must have N >= 1 and K a positive multiple of 128 (N=%lld K=%lld)",
                (long long)N, (long long)K);
  if (M < 1 || M > (1 << 22)) return fail(REC_EINVAL, "q4 gemm: M=%d vectors, 1..%d supported", M, 1 << 22);
  if (!packed || !x || !out || !workspace) return fail(REC_EINVAL, "q4 gemm: null pointer");
  if (out_dtype != REC_BF16 && out_dtype != REC_F32) return fail(REC_EINVAL, "q4 gemm: out dtype must be bf16 or f32");
  if (M > 1 && (x_stride < K || out_stride < N))
    return fail(REC_EINVAL, "q4 gemm: row strides (%lld, %lld) shorter than rows (%lld, %lld)", (long long)x_stride,
                (long long)out_stride, (long long)K, (long long)N);
  if (!aligned16(packed) || !aligned16(x) || !aligned16(workspace) || (M > 1 && x_stride % 8 != 0))
    return fail(REC_EALIGN, "q4 gemm: packed, x and workspace must be 16-byte aligned, x_stride a multiple of 8");
  // a workgroup's 64 rows of x and the packed rows of one tile are addressed
  // through 32-bit buffer offsets
  if ((64 * (M > 1 ? x_stride : K) + K) * 2 >= ((int64_t)1 << 31) || (K / 128) * 1152 >= ((int64_t)1 << 31))
    return fail(REC_EUNSUPPORTED, "q4 gemm: K=%lld, x_stride=%lld exceed the 2 GiB buffer range", (long long)K,
                (long long)x_stride);
  const size_t need = rec_q4_gemm_workspace_bytes(M, K);
  if (workspace_bytes < need)
    return fail(REC_EWORKSPACE, "q4 gemm: workspace of %zu bytes is too small (%zu needed)", workspace_bytes, need);
  Q4GemmArgs a;
  a.packed = (const uint8_t*)packed;
  a.N = N;
  a.K = K;
  a.x = x;
  a.x_stride = M > 1 ? x_stride : K;
  a.M = M;
  a.xsum = (float*)workspace;
  a.out = out;
  a.out_dtype = out_dtype == REC_F32 ? DT_F32 : DT_BF16;
  a.out_stride = out_stride;
  return launched(launch_q4_gemm(a, (hipStream_t)stream), "q4 gemm launch");
}

}  // extern "C"

// ------------------------------------------------------------------------
// Growable KV regions on HIP virtual memory.  A region reserves the address
// range of `rows` rows of `max_tokens` tokens each once, and backs it with
// device memory one bank (bank_tokens tokens of every row) at a time; a
// bank, once mapped, stays at its address until the region is destroyed, so
// growing never copies and every kernel addresses the region as one strided
// tensor (row r at base + r * max_tokens * token_bytes).
namespace {

struct Region {
  int device = 0;
  char* base = nullptr;
  size_t reserved = 0;
  int64_t rows = 0, max_tokens = 0, token_bytes = 0, bank_tokens = 0;
  int banks = 0;                                  // banks mapped so far
  std::vector<hipMemGenericAllocationHandle_t> handles;  // rows x banks, row-major per bank
};

size_t bank_bytes(const Region& r) { return (size_t)r.bank_tokens * (size_t)r.token_bytes; }
char* bank_addr(const Region& r, int64_t row, int bank) {
  return r.base + (size_t)row * (size_t)r.max_tokens * (size_t)r.token_bytes + (size_t)bank * bank_bytes(r);
}

// Unmap and release everything mapped so far, then free the reservation.
void region_release(Region* r) {
  for (int b = 0; b < r->banks; ++b)
    for (int64_t row = 0; row < r->rows; ++row) (void)hipMemUnmap(bank_addr(*r, row, b), bank_bytes(*r));
  for (auto h : r->handles) (void)hipMemRelease(h);
  r->handles.clear();
  r->banks = 0;
  if (r->base) (void)hipMemAddressFree(r->base, r->reserved);
  r->base = nullptr;
}

}  // namespace

extern "C" {

int rec_stream_read(const void* p, int64_t bytes, int workgroups, uint32_t* out, void* stream) {
  if (!p || !out) return fail(REC_EINVAL, "stream read: null pointer");
  if (bytes <= 0 || bytes % 16 != 0) return fail(REC_EINVAL, "stream read: %lld bytes (a positive multiple of 16)",
                                                 (long long)bytes);
  if (!aligned16(p)) return fail(REC_EALIGN, "stream read: the buffer must be 16-byte aligned");
  if (workgroups < 1 || workgroups > 65536) return fail(REC_EINVAL, "stream read: %d workgroups (1..65536)", workgroups);
  return launched(launch_stream_read(p, bytes / 16, workgroups, out, (hipStream_t)stream), "stream read launch");
}

int rec_region_create(int device, int64_t rows, int64_t max_tokens, int64_t token_bytes, int64_t bank_tokens,
                      void** handle, void** base) {
  if (!handle || !base) return fail(REC_EINVAL, "region: null output pointer");
  *handle = nullptr;
  *base = nullptr;
  if (rows < 1 || token_bytes < 1 || bank_tokens < 1 || max_tokens < bank_tokens || max_tokens % bank_tokens != 0)
    return fail(REC_EINVAL, "region: rows %lld, token_bytes %lld, bank_tokens %lld, max_tokens %lld (a multiple of "
                "bank_tokens) must be positive", (long long)rows, (long long)token_bytes, (long long)bank_tokens,
                (long long)max_tokens);
  int vmm = 0;
  hipError_t e = hipDeviceGetAttribute(&vmm, hipDeviceAttributeVirtualMemoryManagementSupported, device);
  if (e != hipSuccess) return fail(REC_EINVAL, "region: device %d: %s", device, hipGetErrorString(e));
  if (!vmm) return fail(REC_EUNSUPPORTED, "region: device %d has no virtual memory management", device);
  hipMemAllocationProp prop{};
  prop.type = hipMemAllocationTypePinned;
  prop.location.type = hipMemLocationTypeDevice;
  prop.location.id = device;
  size_t gran = 0;
  e = hipMemGetAllocationGranularity(&gran, &prop, hipMemAllocationGranularityMinimum);
  if (e != hipSuccess || gran == 0) return fail(REC_ELAUNCH, "region: allocation granularity: %s", hipGetErrorString(e));
  const size_t bank = (size_t)bank_tokens * (size_t)token_bytes;
  if (bank % gran != 0)
    return fail(REC_EINVAL, "region: a bank of %zu bytes per row is not a multiple of the %zu-byte mapping granularity",
                bank, gran);
  Region* r = new Region();
  r->device = device;
  r->rows = rows;
  r->max_tokens = max_tokens;
  r->token_bytes = token_bytes;
  r->bank_tokens = bank_tokens;
  r->reserved = (size_t)rows * (size_t)max_tokens * (size_t)token_bytes;
  void* p = nullptr;
  e = hipMemAddressReserve(&p, r->reserved, gran, nullptr, 0);
  if (e != hipSuccess) {
    size_t n = r->reserved;
    delete r;
    return fail(REC_ELAUNCH, "region: reserving %zu bytes of address space: %s", n, hipGetErrorString(e));
  }
  r->base = (char*)p;
  *handle = r;
  *base = p;
  return ok();
}

int rec_region_grow(void* handle, int64_t tokens, int64_t* capacity) {
  Region* r = (Region*)handle;
  if (!r) return fail(REC_EINVAL, "region: null handle");
  if (tokens < 0 || tokens > r->max_tokens)
    return fail(REC_ECAPACITY, "region: %lld tokens exceed the %lld reserved", (long long)tokens,
                (long long)r->max_tokens);
  const int want = (int)((tokens + r->bank_tokens - 1) / r->bank_tokens);
  hipMemAllocationProp prop{};
  prop.type = hipMemAllocationTypePinned;
  prop.location.type = hipMemLocationTypeDevice;
  prop.location.id = r->device;
  hipMemAccessDesc access{};
  access.location = prop.location;
  access.flags = hipMemAccessFlagsProtReadWrite;
  const size_t bytes = bank_bytes(*r);
  while (r->banks < want) {
    // map bank r->banks of every row; on failure undo this bank's maps
    std::vector<hipMemGenericAllocationHandle_t> made;
    hipError_t e = hipSuccess;
    for (int64_t row = 0; row < r->rows; ++row) {
      hipMemGenericAllocationHandle_t h{};
      if ((e = hipMemCreate(&h, bytes, &prop, 0)) != hipSuccess) break;
      if ((e = hipMemMap(bank_addr(*r, row, r->banks), bytes, 0, h, 0)) != hipSuccess) {
        (void)hipMemRelease(h);
        break;
      }
      made.push_back(h);  // made[k] is mapped at row k
      if ((e = hipMemSetAccess(bank_addr(*r, row, r->banks), bytes, &access, 1)) != hipSuccess) break;
    }
    if (e != hipSuccess) {
      for (int64_t k = 0; k < (int64_t)made.size(); ++k) (void)hipMemUnmap(bank_addr(*r, k, r->banks), bytes);
      for (auto h : made) (void)hipMemRelease(h);
      return fail(REC_ELAUNCH, "region: mapping bank %d (%zu bytes per row, %lld rows): %s", r->banks, bytes,
                  (long long)r->rows, hipGetErrorString(e));
    }
    r->handles.insert(r->handles.end(), made.begin(), made.end());
    ++r->banks;
  }
  if (capacity) *capacity = (int64_t)r->banks * r->bank_tokens;
  return ok();
}

int rec_region_destroy(void* handle) {
  Region* r = (Region*)handle;
  if (!r) return ok();
  region_release(r);
  delete r;
  return ok();
}

}  // extern "C"
