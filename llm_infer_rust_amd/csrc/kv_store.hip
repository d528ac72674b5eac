// Paged K/V store: kc[loc[t]] = k[t], vc[loc[t]] = v[t], bitwise.
//
// Semantics follow the reference write path
//   src/models/attention/base.rs:62-152 (BaseAttention::write_kv)
//   src/models/attention/kv_store.cu:65-99 (sglang_native_store_kv)
//   third_party/sglang/kvcache.cuh:180-211 (store_kvcache: skip reserved slot,
//   require 0 <= slot < capacity)
// The reference aborts the process with a device assert on an out-of-range
// slot. Here the slot is never written and, when the caller passes an
// error-counter word, the count of rejected tokens is added to it so the host
// can turn it into an error without a device trap.
//
// Layout: k/v are [tokens, heads, width] with element strides (kt, kh, 1);
// caches are contiguous [capacity, heads, width] (pages*page_size slots).
#include "common.h"

namespace mi355x {
namespace {

// One thread moves one 16-byte chunk of the K row and the matching chunk of
// the V row. A 2 KiB row (8 heads x 128 x bf16) is 128 threads, so two waves
// cover a token and consecutive lanes touch consecutive addresses.
template <typename Index>
__global__ __launch_bounds__(256) void store_kv_vec(
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, uint16_t* __restrict__ kc,
    uint16_t* __restrict__ vc, const Index* __restrict__ loc, int64_t tokens, int64_t heads,
    int64_t width, int64_t capacity, int64_t kt, int64_t kh, int64_t vt, int64_t vh,
    int64_t reserved, int32_t* __restrict__ error_count) {
  const int64_t chunks_per_head = width >> 3;
  const int64_t chunks = heads * chunks_per_head;
  const int64_t id = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (id >= tokens * chunks) return;
  const int64_t token = id / chunks;
  const int64_t c = id - token * chunks;
  const int64_t slot = static_cast<int64_t>(loc[token]);
  if (slot < 0 || slot >= capacity) {
    if (c == 0 && error_count) atomicAdd(error_count, 1);
    return;
  }
  if (slot == reserved) return;
  const int64_t head = c / chunks_per_head;
  const int64_t col = (c - head * chunks_per_head) << 3;
  const uint4 kval = ld128(k + token * kt + head * kh + col);
  const uint4 vval = ld128(v + token * vt + head * vh + col);
  const int64_t dst = (slot * heads + head) * width + col;
  st128(kc + dst, kval);
  st128(vc + dst, vval);
}

// Any-stride fallback: one 16-bit element per thread.
template <typename Index>
__global__ __launch_bounds__(256) void store_kv_scalar(
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, uint16_t* __restrict__ kc,
    uint16_t* __restrict__ vc, const Index* __restrict__ loc, int64_t tokens, int64_t heads,
    int64_t width, int64_t capacity, int64_t kt, int64_t kh, int64_t vt, int64_t vh,
    int64_t reserved, int32_t* __restrict__ error_count) {
  const int64_t row = heads * width;
  const int64_t id = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (id >= tokens * row) return;
  const int64_t token = id / row;
  const int64_t e = id - token * row;
  const int64_t slot = static_cast<int64_t>(loc[token]);
  if (slot < 0 || slot >= capacity) {
    if (e == 0 && error_count) atomicAdd(error_count, 1);
    return;
  }
  if (slot == reserved) return;
  const int64_t head = e / width;
  const int64_t col = e - head * width;
  kc[slot * row + e] = k[token * kt + head * kh + col];
  vc[slot * row + e] = v[token * vt + head * vh + col];
}

template <typename Index>
void launch(const void* k, const void* v, void* kc, void* vc, const void* loc, int64_t tokens,
            int64_t heads, int64_t width, int64_t capacity, int64_t kt, int64_t kh, int64_t vt,
            int64_t vh, int64_t reserved, int32_t* error_count, bool vec, hipStream_t stream) {
  const auto* kp = static_cast<const uint16_t*>(k);
  const auto* vp = static_cast<const uint16_t*>(v);
  auto* kcp = static_cast<uint16_t*>(kc);
  auto* vcp = static_cast<uint16_t*>(vc);
  const auto* lp = static_cast<const Index*>(loc);
  if (vec) {
    const int64_t threads = tokens * heads * (width / 8);
    const int64_t blocks = (threads + 255) / 256;
    store_kv_vec<Index><<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, stream>>>(
        kp, vp, kcp, vcp, lp, tokens, heads, width, capacity, kt, kh, vt, vh, reserved,
        error_count);
  } else {
    const int64_t threads = tokens * heads * width;
    const int64_t blocks = (threads + 255) / 256;
    store_kv_scalar<Index><<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, stream>>>(
        kp, vp, kcp, vcp, lp, tokens, heads, width, capacity, kt, kh, vt, vh, reserved,
        error_count);
  }
}

}  // namespace
}  // namespace mi355x

using namespace mi355x;

extern "C" const char* mi355x_store_kv(const void* k, const void* v, void* kc, void* vc,
                                       const void* loc, int64_t tokens, int64_t heads,
                                       int64_t width, int64_t capacity, int64_t kt, int64_t kh,
                                       int64_t vt, int64_t vh, int64_t reserved, bool index64,
                                       int32_t* error_count, void* stream) {
  if (tokens < 0 || heads <= 0 || width <= 0 || capacity < 0)
    return set_error("mi355x_store_kv: invalid geometry");
  if (tokens == 0) return nullptr;
  if (!k || !v || !kc || !vc || !loc) return set_error("mi355x_store_kv: null pointer");
  // One thread per element (or per 16-byte chunk); the grid is a single uint32 x
  // dimension of 256-thread blocks, so keep every launch below 2^32 threads.
  if (tokens > (int64_t(1) << 40) / heads || tokens * heads > (int64_t(1) << 40) / width ||
      tokens * heads * width >= (int64_t(1) << 32) - 256)
    return set_error("mi355x_store_kv: launch too large");
  const bool vec = width % 8 == 0 && kt % 8 == 0 && kh % 8 == 0 && vt % 8 == 0 && vh % 8 == 0 &&
                   aligned(k, 16) && aligned(v, 16) && aligned(kc, 16) && aligned(vc, 16);
  auto s = static_cast<hipStream_t>(stream);
  if (index64)
    launch<int64_t>(k, v, kc, vc, loc, tokens, heads, width, capacity, kt, kh, vt, vh, reserved,
                    error_count, vec, s);
  else
    launch<int32_t>(k, v, kc, vc, loc, tokens, heads, width, capacity, kt, kh, vt, vh, reserved,
                    error_count, vec, s);
  return launch_status("mi355x_store_kv");
}
