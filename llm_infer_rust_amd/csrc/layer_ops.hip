// Decoder-layer elementwise ops around attention for gfx950: half-split RoPE,
// the fused QK-norm -> RoPE -> paged K/V store pass, and SiLU(gate) * up.
//
// Numerical contract:
//   rope (src/layers/ops.rs:84-127, fused_ops.cu:108-133): for a head row x of
//     width D, half = D/2, position p (int64) and fp32 tables cos/sin
//     [max_positions, half]:
//       x[i]      <- cast(x[i] * cos[p,i] - x[i+half] * sin[p,i])
//       x[i+half] <- cast(x[i+half] * cos[p,i] + x[i] * sin[p,i])
//     in place for every q and k head; a position outside [0, max_positions)
//     leaves the row untouched (the reference kernel returns early).
//   silu_mul (ops.rs:53-61, fused_ops.cu:135-171): gate_up [T, 2W] contiguous,
//     out[t, c] = cast(silu(gate) * up), silu(g) = g / (1 + exp(-g)).
//   qk_norm_rope_store: the composition qk_norm -> rope -> store_kv that a
//     decoder layer runs (src/models/qwen3/model.rs:478-514), done in one pass
//     over the packed q/k/v rows. The normalised value is rounded to the
//     activation dtype before the rotation, so the result is bit-identical to
//     the three separate launches of this library.
//
// Mapping (D = 128): 16 lanes own one head row, 8 elements per lane (one
// 128-bit access). Lane l holds elements [8l, 8l+8); its rotation partner
// (element i + 64) sits in lane l ^ 8 of the same 16-lane DPP row, so the
// partner values arrive with four row_ror:8 moves of packed words.
#include "common.h"

namespace mi355x {
namespace {

constexpr int kHeadDim = 128;
constexpr int kHalf = kHeadDim / 2;
constexpr int kDppRowRor8 = 0x128;  // row_ror:8 — lane l reads lane (l + 8) mod 16 of its row

__device__ __forceinline__ uint32_t dpp_ror8(uint32_t x) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(x), kDppRowRor8, 0xf, 0xf, false));
}

struct HeadArgs {
  uint16_t* q;
  uint16_t* k;
  const uint16_t* v;
  const uint16_t* qw;  // NULL: no norm
  const uint16_t* kw;
  const int64_t* positions;  // NULL: no rope
  const float* cos;
  const float* sin;
  uint16_t* kc;  // NULL: no store
  uint16_t* vc;
  const void* loc;
  int32_t* error_count;
  int64_t tokens, q_heads, k_heads;
  int64_t qs0, qs1, ks0, ks1, vs0, vs1;
  int64_t max_positions, capacity, reserved;
  float eps;
  // Partials mode: q/k/v rows are the sum of split-K fp32 partials [splits][tokens][ld]
  // (ld = (q_heads + 2 k_heads) * 128), rounded once, and v is written to v_out as well.
  const float* part;
  int64_t part_ld, part_plane;
  int32_t part_splits;
  uint16_t* v_out;
  int64_t vos0, vos1;
};

// One row's 8 columns from the split-K partials: split 0 plus each later split in order (the
// order linear_reduce adds them), rounded once.
template <int DT>
__device__ __forceinline__ uint4 partial_row8(const HeadArgs& a, int64_t token, int64_t col) {
  const float* p = a.part + token * a.part_ld + col;
  float4 lo = *reinterpret_cast<const float4*>(p);
  float4 hi = *reinterpret_cast<const float4*>(p + 4);
  for (int s = 1; s < a.part_splits; ++s) {
    const float4 x = *reinterpret_cast<const float4*>(p + s * a.part_plane);
    const float4 y = *reinterpret_cast<const float4*>(p + s * a.part_plane + 4);
    lo.x += x.x;
    lo.y += x.y;
    lo.z += x.z;
    lo.w += x.w;
    hi.x += y.x;
    hi.y += y.y;
    hi.z += y.z;
    hi.w += y.w;
  }
  const float f[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
  return pack8<DT>(f);
}

// One 16-lane group per (token, head) row, q heads first then k heads.
template <int DT, bool NORM, bool ROPE, bool STORE, typename Index, bool PART = false>
__global__ __launch_bounds__(256) void head_rows_kernel(HeadArgs a) {
  const int lane = threadIdx.x & 15;
  const int64_t per = a.q_heads + a.k_heads;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4);
  if (row >= a.tokens * per) return;  // whole 16-lane group exits together
  const int64_t token = row / per;
  const int64_t h = row - token * per;
  const bool is_q = h < a.q_heads;
  const int64_t kh = h - a.q_heads;
  uint16_t* ptr = is_q ? a.q + token * a.qs0 + h * a.qs1 : a.k + token * a.ks0 + kh * a.ks1;
  ptr += lane * 8;

  uint4 packed;
  uint4 v_packed = make_uint4(0, 0, 0, 0);
  if constexpr (PART) {
    packed = partial_row8<DT>(a, token, h * kHeadDim + lane * 8);
    if (!is_q) {  // the v row of this kv head, kept in the packed output as the reduce would
      v_packed = partial_row8<DT>(a, token, (a.q_heads + a.k_heads + kh) * kHeadDim + lane * 8);
      st128(a.v_out + token * a.vos0 + kh * a.vos1 + lane * 8, v_packed);
    }
  } else {
    packed = ld128(ptr);
  }
  if constexpr (NORM) {
    float x[8];
    unpack8<DT>(packed, x);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = fmaf(x[i], x[i], ss);
    ss = row16_sum(ss);
    const float scale = rsqrtf(ss / static_cast<float>(kHeadDim) + a.eps);
    float w[8];
    unpack8<DT>(ld128((is_q ? a.qw : a.kw) + lane * 8), w);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = (x[i] * scale) * w[i];
    packed = pack8<DT>(x);
  }
  if constexpr (ROPE) {
    const int64_t pos = a.positions[token];
    // The partner exchange is a cross-lane op: every lane of the row takes part.
    uint4 other;
    other.x = dpp_ror8(packed.x);
    other.y = dpp_ror8(packed.y);
    other.z = dpp_ror8(packed.z);
    other.w = dpp_ror8(packed.w);
    if (pos >= 0 && pos < a.max_positions) {
      float mine[8], theirs[8];
      unpack8<DT>(packed, mine);
      unpack8<DT>(other, theirs);
      const int col = (lane & 7) * 8;  // index i within the half
      const float4* cp = reinterpret_cast<const float4*>(a.cos + pos * kHalf + col);
      const float4* sp = reinterpret_cast<const float4*>(a.sin + pos * kHalf + col);
      const float4 c0 = cp[0], c1 = cp[1], s0 = sp[0], s1 = sp[1];
      const float c[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
      const float s[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
      float y[8];
      if (lane < 8) {  // first half: x_i c - x_{i+half} s
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = mine[i] * c[i] - theirs[i] * s[i];
      } else {  // second half: x_{i+half} c + x_i s
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = mine[i] * c[i] + theirs[i] * s[i];
      }
      packed = pack8<DT>(y);
    }
  }
  st128(ptr, packed);

  if constexpr (STORE) {
    if (is_q) return;
    const int64_t slot = static_cast<int64_t>(static_cast<const Index*>(a.loc)[token]);
    if (slot < 0 || slot >= a.capacity) {
      if (kh == 0 && lane == 0 && a.error_count) atomicAdd(a.error_count, 1);
      return;
    }
    if (slot == a.reserved) return;
    const int64_t dst = (slot * a.k_heads + kh) * kHeadDim + lane * 8;
    st128(a.kc + dst, packed);
    st128(a.vc + dst, PART ? v_packed : ld128(a.v + token * a.vs0 + kh * a.vs1 + lane * 8));
  }
}

// Any-width RoPE fallback (one thread per rotated pair), for widths other
// than 128 or unaligned views.
template <int DT>
__global__ __launch_bounds__(256) void rope_scalar_kernel(HeadArgs a, int64_t width) {
  const int64_t half = width / 2;
  const int64_t per = a.q_heads + a.k_heads;
  const int64_t id = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (id >= a.tokens * per * half) return;
  const int64_t row = id / half;
  const int64_t i = id - row * half;
  const int64_t token = row / per;
  const int64_t h = row - token * per;
  const int64_t pos = a.positions[token];
  if (pos < 0 || pos >= a.max_positions) return;
  uint16_t* p = h < a.q_heads ? a.q + token * a.qs0 + h * a.qs1
                              : a.k + token * a.ks0 + (h - a.q_heads) * a.ks1;
  const float first = Elem<DT>::to_float(p[i]);
  const float second = Elem<DT>::to_float(p[i + half]);
  const float c = a.cos[pos * half + i];
  const float s = a.sin[pos * half + i];
  p[i] = Elem<DT>::from_float(first * c - second * s);
  p[i + half] = Elem<DT>::from_float(second * c + first * s);
}

template <int DT, bool NORM, bool ROPE, bool STORE>
void launch_rows(const HeadArgs& a, bool index64, hipStream_t s) {
  const int64_t rows = a.tokens * (a.q_heads + a.k_heads);
  const dim3 grid(static_cast<uint32_t>((rows + 15) / 16));
  if (a.part) {  // the fused QKV path always normalises, rotates and stores
    if constexpr (NORM && ROPE && STORE) {
      if (index64)
        head_rows_kernel<DT, true, true, true, int64_t, true><<<grid, dim3(256), 0, s>>>(a);
      else
        head_rows_kernel<DT, true, true, true, int32_t, true><<<grid, dim3(256), 0, s>>>(a);
    }
    return;
  }
  if (index64)
    head_rows_kernel<DT, NORM, ROPE, STORE, int64_t><<<grid, dim3(256), 0, s>>>(a);
  else
    head_rows_kernel<DT, NORM, ROPE, STORE, int32_t><<<grid, dim3(256), 0, s>>>(a);
}

template <int DT>
void launch_rows_dt(const HeadArgs& a, bool norm, bool rope, bool store, bool index64,
                    hipStream_t s) {
  if (norm && rope && store) return launch_rows<DT, true, true, true>(a, index64, s);
  if (norm && rope) return launch_rows<DT, true, true, false>(a, index64, s);
  if (rope && store) return launch_rows<DT, false, true, true>(a, index64, s);
  if (norm && store) return launch_rows<DT, true, false, true>(a, index64, s);
  if (rope) return launch_rows<DT, false, true, false>(a, index64, s);
  if (norm) return launch_rows<DT, true, false, false>(a, index64, s);
  return launch_rows<DT, false, false, true>(a, index64, s);
}

bool head_views_vectorisable(const HeadArgs& a) {
  return a.qs0 % 8 == 0 && a.qs1 % 8 == 0 && a.ks0 % 8 == 0 && a.ks1 % 8 == 0 &&
         aligned(a.q, 16) && aligned(a.k, 16);
}

// SiLU(gate) * up with one 128-bit chunk of gate, up and out per thread.
template <int DT>
__global__ __launch_bounds__(256) void silu_mul_vec(const uint16_t* __restrict__ gate_up,
                                                    uint16_t* __restrict__ out, int64_t tokens,
                                                    int64_t width) {
  const int64_t chunks = width >> 3;
  const int64_t id = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (id >= tokens * chunks) return;
  const int64_t t = id / chunks;
  const int64_t c = (id - t * chunks) << 3;
  float g[8], u[8], y[8];
  unpack8<DT>(ld128(gate_up + t * 2 * width + c), g);
  unpack8<DT>(ld128(gate_up + t * 2 * width + width + c), u);
#pragma unroll
  for (int i = 0; i < 8; ++i) y[i] = (g[i] / (1.f + __expf(-g[i]))) * u[i];
  st128(out + t * width + c, pack8<DT>(y));
}

template <int DT>
__global__ __launch_bounds__(256) void silu_mul_scalar(const uint16_t* __restrict__ gate_up,
                                                       uint16_t* __restrict__ out,
                                                       int64_t tokens, int64_t width) {
  const int64_t id = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (id >= tokens * width) return;
  const int64_t t = id / width;
  const int64_t c = id - t * width;
  const float g = Elem<DT>::to_float(gate_up[t * 2 * width + c]);
  const float u = Elem<DT>::to_float(gate_up[t * 2 * width + width + c]);
  out[id] = Elem<DT>::from_float((g / (1.f + __expf(-g))) * u);
}

}  // namespace
}  // namespace mi355x

using namespace mi355x;

extern "C" const char* mi355x_rope(void* q, void* k, const int64_t* positions, const float* cos,
                                   const float* sin, int64_t tokens, int64_t q_heads,
                                   int64_t k_heads, int64_t width, int64_t q_token_stride,
                                   int64_t q_head_stride, int64_t k_token_stride,
                                   int64_t k_head_stride, int64_t max_positions, int dtype,
                                   void* stream) {
  if (tokens < 0 || q_heads < 0 || k_heads < 0 || width <= 0 || width % 2 != 0 ||
      max_positions < 0)
    return set_error("mi355x_rope: bad shape");
  if (dtype != 0 && dtype != 1) return set_error("mi355x_rope: dtype must be 0 (bf16) or 1 (fp16)");
  if (tokens == 0 || q_heads + k_heads == 0) return nullptr;
  if (!q || !k || !positions || !cos || !sin) return set_error("mi355x_rope: null pointer");
  HeadArgs a{};
  a.q = static_cast<uint16_t*>(q);
  a.k = static_cast<uint16_t*>(k);
  a.positions = positions;
  a.cos = cos;
  a.sin = sin;
  a.tokens = tokens;
  a.q_heads = q_heads;
  a.k_heads = k_heads;
  a.qs0 = q_token_stride;
  a.qs1 = q_head_stride;
  a.ks0 = k_token_stride;
  a.ks1 = k_head_stride;
  a.max_positions = max_positions;
  auto s = static_cast<hipStream_t>(stream);
  if (width == kHeadDim && head_views_vectorisable(a) && aligned(cos, 16) && aligned(sin, 16)) {
    if (dtype == 0)
      launch_rows_dt<0>(a, false, true, false, false, s);
    else
      launch_rows_dt<1>(a, false, true, false, false, s);
  } else {
    const int64_t threads = tokens * (q_heads + k_heads) * (width / 2);
    const dim3 grid(static_cast<uint32_t>((threads + 255) / 256));
    if (dtype == 0)
      rope_scalar_kernel<0><<<grid, dim3(256), 0, s>>>(a, width);
    else
      rope_scalar_kernel<1><<<grid, dim3(256), 0, s>>>(a, width);
  }
  return launch_status("mi355x_rope");
}

namespace {
// The QK-norm -> RoPE -> K/V store pass; with `part` its q/k/v rows come from split-K
// partials (see HeadArgs) and v is also written to `v_out` (same strides as v). With
// `check_only` it validates the arguments and launches nothing.
const char* qk_rows_impl(
    void* q, void* k, const void* v, const void* q_weight, const void* k_weight,
    const int64_t* positions, const float* cos, const float* sin, int64_t max_positions,
    void* k_cache, void* v_cache, const void* loc, bool index64, int64_t capacity,
    int64_t reserved, int32_t* error_count, int64_t tokens, int64_t q_heads, int64_t k_heads,
    int64_t width, int64_t q_token_stride, int64_t q_head_stride, int64_t k_token_stride,
    int64_t k_head_stride, int64_t v_token_stride, int64_t v_head_stride, double eps, int dtype,
    void* stream, const float* part, int32_t part_splits, bool check_only = false) {
  if (tokens < 0 || q_heads < 0 || k_heads < 0 || max_positions < 0 || capacity < 0)
    return set_error("mi355x_qk_norm_rope_store: bad shape");
  if (width != kHeadDim) return set_error("mi355x_qk_norm_rope_store: width must be 128");
  if (dtype != 0 && dtype != 1)
    return set_error("mi355x_qk_norm_rope_store: dtype must be 0 (bf16) or 1 (fp16)");
  const bool norm = q_weight != nullptr || k_weight != nullptr;
  const bool rope = positions != nullptr;
  const bool store = k_cache != nullptr;
  if (norm && (!q_weight || !k_weight))
    return set_error("mi355x_qk_norm_rope_store: q_weight and k_weight go together");
  if (rope && (!cos || !sin)) return set_error("mi355x_qk_norm_rope_store: cos/sin missing");
  if (store && (!v_cache || !loc || !v))
    return set_error("mi355x_qk_norm_rope_store: store needs v, v_cache and loc");
  if (!norm && !rope && !store) return nullptr;
  if (tokens == 0 || q_heads + k_heads == 0) return nullptr;
  if (!q || !k) return set_error("mi355x_qk_norm_rope_store: null q/k");
  HeadArgs a{};
  a.q = static_cast<uint16_t*>(q);
  a.k = static_cast<uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.qw = static_cast<const uint16_t*>(q_weight);
  a.kw = static_cast<const uint16_t*>(k_weight);
  a.positions = positions;
  a.cos = cos;
  a.sin = sin;
  a.kc = static_cast<uint16_t*>(k_cache);
  a.vc = static_cast<uint16_t*>(v_cache);
  a.loc = loc;
  a.error_count = error_count;
  a.tokens = tokens;
  a.q_heads = q_heads;
  a.k_heads = k_heads;
  a.qs0 = q_token_stride;
  a.qs1 = q_head_stride;
  a.ks0 = k_token_stride;
  a.ks1 = k_head_stride;
  a.vs0 = v_token_stride;
  a.vs1 = v_head_stride;
  a.max_positions = max_positions;
  a.capacity = capacity;
  a.reserved = reserved;
  a.eps = static_cast<float>(eps);
  if (part) {
    if (!(norm && rope && store) || part_splits < 2 || !aligned(part, 16))
      return set_error("mi355x_linear_qk_norm_rope_store: needs norm weights, positions and a cache");
    a.part = part;
    a.part_splits = part_splits;
    a.part_ld = (q_heads + 2 * k_heads) * kHeadDim;
    a.part_plane = tokens * a.part_ld;
    a.v_out = static_cast<uint16_t*>(const_cast<void*>(v));
    a.vos0 = v_token_stride;
    a.vos1 = v_head_stride;
  }
  bool ok = head_views_vectorisable(a);
  if (norm) ok = ok && aligned(q_weight, 16) && aligned(k_weight, 16);
  if (rope) ok = ok && aligned(cos, 16) && aligned(sin, 16);
  if (store)
    ok = ok && v_token_stride % 8 == 0 && v_head_stride % 8 == 0 && aligned(v, 16) &&
         aligned(k_cache, 16) && aligned(v_cache, 16);
  if (!ok)
    return set_error(
        "mi355x_qk_norm_rope_store: views must be 16-byte aligned with strides divisible by 8");
  if (check_only) return nullptr;
  auto s = static_cast<hipStream_t>(stream);
  if (dtype == 0)
    launch_rows_dt<0>(a, norm, rope, store, index64, s);
  else
    launch_rows_dt<1>(a, norm, rope, store, index64, s);
  return launch_status("mi355x_qk_norm_rope_store");
}
}  // namespace

extern "C" const char* mi355x_qk_norm_rope_store(
    void* q, void* k, const void* v, const void* q_weight, const void* k_weight,
    const int64_t* positions, const float* cos, const float* sin, int64_t max_positions,
    void* k_cache, void* v_cache, const void* loc, bool index64, int64_t capacity,
    int64_t reserved, int32_t* error_count, int64_t tokens, int64_t q_heads, int64_t k_heads,
    int64_t width, int64_t q_token_stride, int64_t q_head_stride, int64_t k_token_stride,
    int64_t k_head_stride, int64_t v_token_stride, int64_t v_head_stride, double eps, int dtype,
    void* stream) {
  return qk_rows_impl(q, k, v, q_weight, k_weight, positions, cos, sin, max_positions, k_cache,
                      v_cache, loc, index64, capacity, reserved, error_count, tokens, q_heads,
                      k_heads, width, q_token_stride, q_head_stride, k_token_stride,
                      k_head_stride, v_token_stride, v_head_stride, eps, dtype, stream, nullptr,
                      0);
}

extern "C" const char* mi355x_linear_qk_norm_rope_store(
    const void* x, int64_t ldx, const void* w, int64_t ldw, void* qkv, int64_t ldo, int64_t M,
    int64_t K, int64_t q_heads, int64_t k_heads, void* workspace, int64_t workspace_bytes,
    int32_t cus, const void* q_weight, const void* k_weight, const int64_t* positions,
    const float* cos, const float* sin, int64_t max_positions, void* k_cache, void* v_cache,
    const void* loc, bool index64, int64_t capacity, int64_t reserved, int32_t* error_count,
    double eps, int dtype, void* stream) {
  if (M <= 0 || q_heads <= 0 || k_heads <= 0 || ldo % 8 || !qkv || !aligned(qkv, 16))
    return set_error("mi355x_linear_qk_norm_rope_store: bad shape");
  if (!q_weight || !k_weight || !positions || !k_cache)
    return set_error("mi355x_linear_qk_norm_rope_store: needs norm weights, positions and a cache");
  const int64_t N = (q_heads + 2 * k_heads) * kHeadDim;
  if (ldo < N) return set_error("mi355x_linear_qk_norm_rope_store: ldo < (Hq + 2 Hkv) * 128");
  if (workspace && !aligned(workspace, 16))
    return set_error("mi355x_linear_qk_norm_rope_store: workspace must be 16-byte aligned");
  auto* base = static_cast<uint16_t*>(qkv);
  // Every argument of the pass is checked before the projection is queued, so a refused
  // call launches nothing (and leaves no unreduced split-K partials behind).
  if (const char* e = qk_rows_impl(
          base, base + q_heads * kHeadDim, base + (q_heads + k_heads) * kHeadDim, q_weight,
          k_weight, positions, cos, sin, max_positions, k_cache, v_cache, loc, index64,
          capacity, reserved, error_count, M, q_heads, k_heads, kHeadDim, ldo, kHeadDim, ldo,
          kHeadDim, ldo, kHeadDim, eps, dtype, stream, nullptr, 0, true))
    return e;
  auto s = static_cast<hipStream_t>(stream);
  int used = 1;
  if (const char* e = run_linear(x, ldx, w, ldw, qkv, ldo, M, N, K, workspace, workspace_bytes,
                                 cus, -1, -1, dtype, true, &used, s))
    return e;
  return qk_rows_impl(base, base + q_heads * kHeadDim, base + (q_heads + k_heads) * kHeadDim,
                      q_weight, k_weight, positions, cos, sin, max_positions, k_cache, v_cache,
                      loc, index64, capacity, reserved, error_count, M, q_heads, k_heads,
                      kHeadDim, ldo, kHeadDim, ldo, kHeadDim, ldo, kHeadDim, eps, dtype, stream,
                      used > 1 ? static_cast<const float*>(workspace) : nullptr, used);
}

extern "C" const char* mi355x_silu_mul(const void* gate_up, void* out, int64_t tokens,
                                       int64_t width, int dtype, void* stream) {
  if (tokens < 0 || width <= 0) return set_error("mi355x_silu_mul: bad shape");
  if (dtype != 0 && dtype != 1)
    return set_error("mi355x_silu_mul: dtype must be 0 (bf16) or 1 (fp16)");
  if (tokens == 0) return nullptr;
  if (!gate_up || !out) return set_error("mi355x_silu_mul: null pointer");
  auto s = static_cast<hipStream_t>(stream);
  const auto* in = static_cast<const uint16_t*>(gate_up);
  auto* o = static_cast<uint16_t*>(out);
  if (width % 8 == 0 && aligned(gate_up, 16) && aligned(out, 16)) {
    const int64_t threads = tokens * (width / 8);
    const dim3 grid(static_cast<uint32_t>((threads + 255) / 256));
    if (dtype == 0)
      silu_mul_vec<0><<<grid, dim3(256), 0, s>>>(in, o, tokens, width);
    else
      silu_mul_vec<1><<<grid, dim3(256), 0, s>>>(in, o, tokens, width);
  } else {
    const int64_t threads = tokens * width;
    const dim3 grid(static_cast<uint32_t>((threads + 255) / 256));
    if (dtype == 0)
      silu_mul_scalar<0><<<grid, dim3(256), 0, s>>>(in, o, tokens, width);
    else
      silu_mul_scalar<1><<<grid, dim3(256), 0, s>>>(in, o, tokens, width);
  }
  return launch_status("mi355x_silu_mul");
}
