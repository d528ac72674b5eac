// RMSNorm, fused residual-add RMSNorm and per-head QK-norm for gfx950.
//
// Numerical contract (src/layers/ops.rs:8-51):
//   rms_norm:      y = cast(x_f32 * rsqrt(mean(x_f32^2) + eps) * w_f32)
//   add_rms_norm:  s = x_f32 + r_f32; r <- cast(s); x <- cast(rms(s) * w)
//                  (normalisation uses the UNROUNDED fp32 sum)
//   qk_norm:       rms_norm of every q head with q_w and every k head with k_w,
//                  in place; V bytes are never touched.
// Entry points mirror the reference raw launchers
//   sglang_layers_native_norm / _add_norm / _qk_norm (src/layers/fused_ops.cu:210-338).
//
// Mapping: a row (one token, or one (token, head)) is owned by a group of
// LPR lanes (16 or 64). Each lane keeps NCH 128-bit chunks of the row in
// registers, so HBM sees exactly one read and one write of every byte. The
// sum of squares is reduced with DPP row operations (16 lanes) plus two
// cross-row shuffles for 64-lane rows.
#include "common.h"

namespace mi355x {
namespace {

enum NormMode { kRms = 0, kAddRms = 1, kQk = 2 };

struct NormArgs {
  // kRms: x (read), out (write). kAddRms: x, residual (both read+write).
  // kQk: x = q, residual = k (both in place); weight = q_w, weight2 = k_w.
  uint16_t* x;
  uint16_t* residual;
  uint16_t* out;
  const uint16_t* weight;
  const uint16_t* weight2;
  int64_t rows;
  int64_t heads;   // kRms: heads per token; kQk: q heads
  int64_t heads2;  // kQk: k heads
  int64_t width;
  int64_t xs0, xs1;  // token / head stride of x (or q)
  int64_t rs0, rs1;  // token / head stride of residual (or k)
  float eps;
};

template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (LPR == 16) {
    return row16_sum(v);
  } else {
    return wave_sum(v);
  }
}

// Resolve a row index into (source pointer, destination pointer, weight).
template <int MODE>
__device__ __forceinline__ void row_pointers(const NormArgs& a, int64_t row, uint16_t*& src,
                                             uint16_t*& dst, uint16_t*& res,
                                             const uint16_t*& w) {
  if constexpr (MODE == kRms) {
    const int64_t token = row / a.heads;
    const int64_t head = row - token * a.heads;
    src = a.x + token * a.xs0 + head * a.xs1;
    dst = a.out + row * a.width;
    res = nullptr;
    w = a.weight;
  } else if constexpr (MODE == kAddRms) {
    src = a.x + row * a.xs0;
    dst = src;
    res = a.residual + row * a.rs0;
    w = a.weight;
  } else {
    const int64_t per = a.heads + a.heads2;
    const int64_t token = row / per;
    const int64_t h = row - token * per;
    if (h < a.heads) {
      src = a.x + token * a.xs0 + h * a.xs1;
      w = a.weight;
    } else {
      src = a.residual + token * a.rs0 + (h - a.heads) * a.rs1;
      w = a.weight2;
    }
    dst = src;
    res = nullptr;
  }
}

// Vectorised row kernel: requires width % 8 == 0, 16-byte aligned rows and
// width <= LPR * 8 * NCH.
template <int DT, int MODE, int LPR, int NCH>
__global__ __launch_bounds__(256) void norm_vec(NormArgs a) {
  constexpr int kGroups = 256 / LPR;
  const int lane = threadIdx.x % LPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kGroups + threadIdx.x / LPR;
  if (row >= a.rows) return;  // whole group exits together: reductions stay in-group
  uint16_t *src, *dst, *res;
  const uint16_t* w;
  row_pointers<MODE>(a, row, src, dst, res, w);
  const int chunks = static_cast<int>(a.width >> 3);

  float vals[NCH][8];
  uint4 wraw[NCH];  // weights issued with the row, off the reduction's critical path
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int chunk = lane + c * LPR;
    if (chunk < chunks) wraw[c] = ld128(w + chunk * 8);
  }
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int chunk = lane + c * LPR;
    if (chunk < chunks) {
      unpack8<DT>(ld128(src + chunk * 8), vals[c]);
      if constexpr (MODE == kAddRms) {
        float r[8];
        unpack8<DT>(ld128(res + chunk * 8), r);
#pragma unroll
        for (int i = 0; i < 8; ++i) vals[c][i] += r[i];
        st128(res + chunk * 8, pack8<DT>(vals[c]));
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = fmaf(vals[c][i], vals[c][i], ss);
    }
  }
  ss = group_sum<LPR>(ss);
  const float scale = rsqrtf(ss / static_cast<float>(a.width) + a.eps);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int chunk = lane + c * LPR;
    if (chunk < chunks) {
      float wf[8];
      unpack8<DT>(wraw[c], wf);
      float y[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = (vals[c][i] * scale) * wf[i];
      st128(dst + chunk * 8, pack8<DT>(y));
    }
  }
}

// Narrow rows (one 128-element head or less), RPT rows per 16-lane group: the group's rows
// sit 16 groups apart, all RPT row loads (and weights) are issued before the first
// reduction, so each lane keeps RPT 16-byte loads in flight instead of one. Rows past the
// end are masked per group (the group's 16 lanes share a row, so the DPP sums stay in it).
template <int DT, int MODE, int RPT>
__global__ __launch_bounds__(256) void norm_vec16_rows(NormArgs a) {
  const int lane = threadIdx.x & 15;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * 16 * RPT + (threadIdx.x >> 4);
  const int chunks = static_cast<int>(a.width >> 3);
  const bool lane_on = lane < chunks;
  uint16_t* src[RPT];
  uint16_t* dst[RPT];
  uint4 raw[RPT], wraw[RPT];
  bool ok[RPT];
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const int64_t row = row0 + 16 * k;
    ok[k] = row < a.rows;
    uint16_t* res;
    const uint16_t* w;
    row_pointers<MODE>(a, ok[k] ? row : 0, src[k], dst[k], res, w);
    if (ok[k] && lane_on) {
      wraw[k] = ld128(w + lane * 8);
      raw[k] = ld128(src[k] + lane * 8);
    }
  }
  float ss[RPT];
  float vals[RPT][8];
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    ss[k] = 0.f;
    if (ok[k] && lane_on) {
      unpack8<DT>(raw[k], vals[k]);
#pragma unroll
      for (int i = 0; i < 8; ++i) ss[k] = fmaf(vals[k][i], vals[k][i], ss[k]);
    }
  }
  row16_sum_n<RPT>(ss);
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    if (ok[k] && lane_on) {
      const float scale = rsqrtf(ss[k] / static_cast<float>(a.width) + a.eps);
      float wf[8];
      unpack8<DT>(wraw[k], wf);
      float y[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = (vals[k][i] * scale) * wf[i];
      st128(dst[k] + lane * 8, pack8<DT>(y));
    }
  }
}

// Many rows, RPT rows per LPR-lane group: a group's rows sit (256 / LPR) groups apart and
// all RPT rows' loads (data and weights) are issued before the first reduction, so each
// lane keeps RPT times as many 16-byte loads in flight as one row allows. Rows past the end
// are masked per group (the group's lanes share a row, so the reductions stay in it).
template <int DT, int MODE, int LPR, int NCH, int RPT>
__global__ __launch_bounds__(256) void norm_vec_rows(NormArgs a) {
  constexpr int kGroups = 256 / LPR;
  const int lane = threadIdx.x % LPR;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kGroups * RPT + threadIdx.x / LPR;
  const int chunks = static_cast<int>(a.width >> 3);
  uint16_t* dst[RPT];
  uint16_t* res[RPT];
  uint4 raw[RPT][NCH], wraw[RPT][NCH], rraw[RPT][NCH];
  bool ok[RPT];
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const int64_t row = row0 + kGroups * k;
    ok[k] = row < a.rows;
    uint16_t* src;
    const uint16_t* w;
    row_pointers<MODE>(a, ok[k] ? row : 0, src, dst[k], res[k], w);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int chunk = lane + c * LPR;
      if (ok[k] && chunk < chunks) {
        wraw[k][c] = ld128(w + chunk * 8);
        raw[k][c] = ld128(src + chunk * 8);
        if constexpr (MODE == kAddRms) rraw[k][c] = ld128(res[k] + chunk * 8);
      }
    }
  }
  float ss[RPT];
  float vals[RPT][NCH][8];
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    ss[k] = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int chunk = lane + c * LPR;
      if (ok[k] && chunk < chunks) {
        unpack8<DT>(raw[k][c], vals[k][c]);
        if constexpr (MODE == kAddRms) {
          float r[8];
          unpack8<DT>(rraw[k][c], r);
#pragma unroll
          for (int i = 0; i < 8; ++i) vals[k][c][i] += r[i];
          st128(res[k] + chunk * 8, pack8<DT>(vals[k][c]));
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) ss[k] = fmaf(vals[k][c][i], vals[k][c][i], ss[k]);
      }
    }
  }
  if constexpr (LPR == 16) {
    row16_sum_n<RPT>(ss);
  } else {
#pragma unroll
    for (int k = 0; k < RPT; ++k) ss[k] = wave_sum(ss[k]);
  }
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const float scale = rsqrtf(ss[k] / static_cast<float>(a.width) + a.eps);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int chunk = lane + c * LPR;
      if (ok[k] && chunk < chunks) {
        float wf[8];
        unpack8<DT>(wraw[k][c], wf);
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = (vals[k][c][i] * scale) * wf[i];
        st128(dst[k] + chunk * 8, pack8<DT>(y));
      }
    }
  }
}

// Few wide rows (decode-size batches of hidden rows): one 256-lane workgroup per
// row so a batch of a few hundred rows still spreads over every CU. Each lane
// holds NCH 128-bit chunks; the sum of squares crosses waves through LDS.
template <int DT, int MODE, int NCH>
__global__ __launch_bounds__(256) void norm_row_block(NormArgs a) {
  __shared__ float partial[4];
  const int64_t row = blockIdx.x;
  uint16_t *src, *dst, *res;
  const uint16_t* w;
  row_pointers<MODE>(a, row, src, dst, res, w);
  const int chunks = static_cast<int>(a.width >> 3);
  float vals[NCH][8];
  uint4 wraw[NCH];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int chunk = threadIdx.x + c * 256;
    if (chunk < chunks) wraw[c] = ld128(w + chunk * 8);
  }
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int chunk = threadIdx.x + c * 256;
    if (chunk < chunks) {
      unpack8<DT>(ld128(src + chunk * 8), vals[c]);
      if constexpr (MODE == kAddRms) {
        float r[8];
        unpack8<DT>(ld128(res + chunk * 8), r);
#pragma unroll
        for (int i = 0; i < 8; ++i) vals[c][i] += r[i];
        st128(res + chunk * 8, pack8<DT>(vals[c]));
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = fmaf(vals[c][i], vals[c][i], ss);
    }
  }
  ss = wave_sum(ss);
  if (threadIdx.x % kWave == 0) partial[threadIdx.x / kWave] = ss;
  __syncthreads();
  ss = (partial[0] + partial[1]) + (partial[2] + partial[3]);
  const float scale = rsqrtf(ss / static_cast<float>(a.width) + a.eps);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int chunk = threadIdx.x + c * 256;
    if (chunk < chunks) {
      float wf[8];
      unpack8<DT>(wraw[c], wf);
      float y[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = (vals[c][i] * scale) * wf[i];
      st128(dst + chunk * 8, pack8<DT>(y));
    }
  }
}

// Generic kernel for any width/stride/alignment: one wave per row, scalar
// elements, two passes (the second pass re-reads the row from cache).
template <int DT, int MODE>
__global__ __launch_bounds__(256) void norm_scalar(NormArgs a) {
  const int lane = threadIdx.x % kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
  if (row >= a.rows) return;
  uint16_t *src, *dst, *res;
  const uint16_t* w;
  row_pointers<MODE>(a, row, src, dst, res, w);
  float ss = 0.f;
  for (int64_t i = lane; i < a.width; i += kWave) {
    float x = Elem<DT>::to_float(src[i]);
    if constexpr (MODE == kAddRms) x += Elem<DT>::to_float(res[i]);
    ss = fmaf(x, x, ss);
  }
  ss = wave_sum(ss);
  const float scale = rsqrtf(ss / static_cast<float>(a.width) + a.eps);
  for (int64_t i = lane; i < a.width; i += kWave) {
    float x = Elem<DT>::to_float(src[i]);
    if constexpr (MODE == kAddRms) {
      x += Elem<DT>::to_float(res[i]);
      res[i] = Elem<DT>::from_float(x);
    }
    dst[i] = Elem<DT>::from_float((x * scale) * Elem<DT>::to_float(w[i]));
  }
}

// Rows per 16-lane group for narrow rows (QK-norm over 8192 x 24 heads: 1 row 25.3 us,
// 2 rows 20.2, 4 rows 21.9, 8 rows 24.2).
constexpr int kNarrowRows = 2;

template <int DT, int MODE>
const char* dispatch(const NormArgs& a, bool vec, hipStream_t s, const char* name) {
  if (a.rows == 0) return nullptr;
  const int64_t chunks = a.width / 8;
  if (vec && chunks <= 16 && MODE != kAddRms && a.rows >= 16 * kNarrowRows * 1024) {
    // <= 128 elements, many rows: 16 lanes per row, kNarrowRows rows per lane group.
    const int64_t blocks = (a.rows + 16 * kNarrowRows - 1) / (16 * kNarrowRows);
    norm_vec16_rows<DT, MODE, kNarrowRows>
        <<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, s>>>(a);
    return launch_status(name);
  }
  if (vec && MODE == kRms && chunks > 64 && chunks <= 128) {
    // 513..1024 elements, no residual: one wave per row, both chunks' loads up front.
    const int64_t blocks = (a.rows + 3) / 4;
    norm_vec_rows<DT, MODE, 64, 2, 1>
        <<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, s>>>(a);
    return launch_status(name);
  }
  if (vec && chunks <= 16) {  // <= 128 elements: 16 lanes per row, 16 rows per block
    const int64_t blocks = (a.rows + 15) / 16;
    norm_vec<DT, MODE, 16, 1><<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, s>>>(a);
    return launch_status(name);
  }
  if (vec && chunks <= 32) {
    const int64_t blocks = (a.rows + 15) / 16;
    norm_vec<DT, MODE, 16, 2><<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, s>>>(a);
    return launch_status(name);
  }
  // Wide rows, too few of them to give every CU four rows: a workgroup per row.
  if (vec && chunks > 128 && chunks <= 256 * 4 && a.rows < 4 * 256 * 4) {
    const dim3 grid(static_cast<uint32_t>(a.rows));
    if (chunks <= 256)
      norm_row_block<DT, MODE, 1><<<grid, dim3(256), 0, s>>>(a);
    else if (chunks <= 512)
      norm_row_block<DT, MODE, 2><<<grid, dim3(256), 0, s>>>(a);
    else
      norm_row_block<DT, MODE, 4><<<grid, dim3(256), 0, s>>>(a);
    return launch_status(name);
  }
  if (vec && chunks <= 64 * 8) {
    const int64_t blocks = (a.rows + 3) / 4;
    const dim3 grid(static_cast<uint32_t>(blocks));
    if (chunks <= 64)
      norm_vec<DT, MODE, 64, 1><<<grid, dim3(256), 0, s>>>(a);
    else if (chunks <= 128)
      norm_vec<DT, MODE, 64, 2><<<grid, dim3(256), 0, s>>>(a);
    else if (chunks <= 256)
      norm_vec<DT, MODE, 64, 4><<<grid, dim3(256), 0, s>>>(a);
    else
      norm_vec<DT, MODE, 64, 8><<<grid, dim3(256), 0, s>>>(a);
    return launch_status(name);
  }
  const int64_t blocks = (a.rows + 3) / 4;
  norm_scalar<DT, MODE><<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, s>>>(a);
  return launch_status(name);
}

template <int MODE>
const char* dispatch_dtype(const NormArgs& a, int dtype, bool vec, hipStream_t s,
                           const char* name) {
  if (dtype == 0) return dispatch<0, MODE>(a, vec, s, name);
  if (dtype == 1) return dispatch<1, MODE>(a, vec, s, name);
  return set_error(std::string(name) + ": dtype must be 0 (bf16) or 1 (fp16)");
}

}  // namespace
}  // namespace mi355x

using namespace mi355x;

extern "C" const char* mi355x_rms_norm(const void* x, const void* weight, void* out,
                                       int64_t tokens, int64_t heads, int64_t width,
                                       int64_t token_stride, int64_t head_stride, double eps,
                                       int dtype, void* stream) {
  if (tokens < 0 || heads <= 0 || width <= 0) return set_error("mi355x_rms_norm: bad shape");
  if (tokens == 0) return nullptr;
  if (!x || !weight || !out) return set_error("mi355x_rms_norm: null pointer");
  NormArgs a{};
  a.x = const_cast<uint16_t*>(static_cast<const uint16_t*>(x));
  a.out = static_cast<uint16_t*>(out);
  a.weight = static_cast<const uint16_t*>(weight);
  a.rows = tokens * heads;
  a.heads = heads;
  a.width = width;
  a.xs0 = token_stride;
  a.xs1 = head_stride;
  a.eps = static_cast<float>(eps);
  const bool vec = width % 8 == 0 && token_stride % 8 == 0 && (heads == 1 || head_stride % 8 == 0) &&
                   aligned(x, 16) && aligned(weight, 16) && aligned(out, 16);
  return dispatch_dtype<kRms>(a, dtype, vec, static_cast<hipStream_t>(stream), "mi355x_rms_norm");
}

extern "C" const char* mi355x_add_rms_norm(void* x, void* residual, const void* weight,
                                           int64_t tokens, int64_t width, int64_t x_stride,
                                           int64_t residual_stride, double eps, int dtype,
                                           void* stream) {
  if (tokens < 0 || width <= 0) return set_error("mi355x_add_rms_norm: bad shape");
  if (tokens == 0) return nullptr;
  if (!x || !residual || !weight) return set_error("mi355x_add_rms_norm: null pointer");
  if (x == residual) return set_error("mi355x_add_rms_norm: x and residual must not alias");
  NormArgs a{};
  a.x = static_cast<uint16_t*>(x);
  a.residual = static_cast<uint16_t*>(residual);
  a.weight = static_cast<const uint16_t*>(weight);
  a.rows = tokens;
  a.heads = 1;
  a.width = width;
  a.xs0 = x_stride;
  a.rs0 = residual_stride;
  a.eps = static_cast<float>(eps);
  const bool vec = width % 8 == 0 && x_stride % 8 == 0 && residual_stride % 8 == 0 &&
                   aligned(x, 16) && aligned(residual, 16) && aligned(weight, 16);
  return dispatch_dtype<kAddRms>(a, dtype, vec, static_cast<hipStream_t>(stream),
                                 "mi355x_add_rms_norm");
}

extern "C" const char* mi355x_qk_norm(void* q, void* k, const void* q_weight,
                                      const void* k_weight, int64_t tokens, int64_t q_heads,
                                      int64_t k_heads, int64_t width, int64_t q_token_stride,
                                      int64_t q_head_stride, int64_t k_token_stride,
                                      int64_t k_head_stride, double eps, int dtype,
                                      void* stream) {
  if (tokens < 0 || q_heads < 0 || k_heads < 0 || width <= 0)
    return set_error("mi355x_qk_norm: bad shape");
  if (tokens == 0 || q_heads + k_heads == 0) return nullptr;
  if ((q_heads && (!q || !q_weight)) || (k_heads && (!k || !k_weight)))
    return set_error("mi355x_qk_norm: null pointer");
  NormArgs a{};
  a.x = static_cast<uint16_t*>(q);
  a.residual = static_cast<uint16_t*>(k);
  a.weight = static_cast<const uint16_t*>(q_weight);
  a.weight2 = static_cast<const uint16_t*>(k_weight);
  a.rows = tokens * (q_heads + k_heads);
  a.heads = q_heads;
  a.heads2 = k_heads;
  a.width = width;
  a.xs0 = q_token_stride;
  a.xs1 = q_head_stride;
  a.rs0 = k_token_stride;
  a.rs1 = k_head_stride;
  a.eps = static_cast<float>(eps);
  const bool vec = width % 8 == 0 && q_token_stride % 8 == 0 && q_head_stride % 8 == 0 &&
                   k_token_stride % 8 == 0 && k_head_stride % 8 == 0 && aligned(q, 16) &&
                   aligned(k, 16) && aligned(q_weight, 16) && aligned(k_weight, 16);
  return dispatch_dtype<kQk>(a, dtype, vec, static_cast<hipStream_t>(stream), "mi355x_qk_norm");
}
