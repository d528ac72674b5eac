// Shared device/host helpers for the gfx950 attention hot path.
//
// Element types are carried as raw 16-bit words (uint16_t). dtype code 0 is
// bfloat16 and 1 is float16, the same codes the reference server passes
// through its native ABI (src/models/attention/flashinfer_bridge.cpp:81,
// src/layers/fused_ops.cu:210-213).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "mi355x_attn.h"

namespace mi355x {

constexpr int kWave = 64;  // CDNA wavefront width

// ----------------------------------------------------------------------------
// Error plumbing: every raw entry point returns NULL on success, otherwise a
// pointer to a thread-local message that stays valid until the next failing
// call on the same thread.
// ----------------------------------------------------------------------------
const char* set_error(const std::string& message);
const char* hip_error(hipError_t status, const char* what);
const char* launch_status(const char* what);

inline bool aligned(const void* p, uintptr_t a) {
  return reinterpret_cast<uintptr_t>(p) % a == 0;
}

// ----------------------------------------------------------------------------
// 16-bit float conversions. bf16 -> f32 is exact (shift); f32 -> bf16/f16
// rounds to nearest-even, which is what torch's CPU and GPU casts do, so
// residual write-backs compare bit-exactly.
// ----------------------------------------------------------------------------
template <int DT>
struct Elem;

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_vec_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_vec_t __attribute__((ext_vector_type(2)));

// Conversions use the gfx950 hardware converts (v_cvt_pk_bf16_f32 /
// v_cvt_f16_f32), which round to nearest-even.
template <>
struct Elem<0> {  // bfloat16
  __device__ __forceinline__ static float to_float(uint16_t h) {
    return __uint_as_float(static_cast<uint32_t>(h) << 16);
  }
  __device__ __forceinline__ static uint16_t from_float(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
  }
  // Two floats -> one packed word {lo = a, hi = b}.
  __device__ __forceinline__ static uint32_t pack2(float a, float b) {
    const f32x2_t v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_vec_t));
  }
};

template <>
struct Elem<1> {  // float16
  __device__ __forceinline__ static float to_float(uint16_t h) {
    _Float16 v = __builtin_bit_cast(_Float16, h);
    return static_cast<float>(v);
  }
  __device__ __forceinline__ static uint16_t from_float(float f) {
    _Float16 v = static_cast<_Float16>(f);  // round-to-nearest-even
    return __builtin_bit_cast(uint16_t, v);
  }
  __device__ __forceinline__ static uint32_t pack2(float a, float b) {
    const f32x2_t v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_vec_t));
  }
};

// Unpack 8 packed 16-bit values (one 128-bit load) into floats.
template <int DT>
__device__ __forceinline__ void unpack8(const uint4& w, float (&f)[8]) {
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = Elem<DT>::to_float(static_cast<uint16_t>(words[i] & 0xffffu));
    f[2 * i + 1] = Elem<DT>::to_float(static_cast<uint16_t>(words[i] >> 16));
  }
}

template <int DT>
__device__ __forceinline__ uint4 pack8(const float (&f)[8]) {
  return make_uint4(Elem<DT>::pack2(f[0], f[1]), Elem<DT>::pack2(f[2], f[3]),
                    Elem<DT>::pack2(f[4], f[5]), Elem<DT>::pack2(f[6], f[7]));
}

// ----------------------------------------------------------------------------
// Cross-lane reductions built on DPP row operations. A DPP "row" is 16 lanes,
// so a 16-lane sum needs four register-to-register steps and no LDS traffic:
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror.
// Every lane of the row ends up holding the row total.
// ----------------------------------------------------------------------------
constexpr int kDppQuadSwap1 = 0xB1;      // quad_perm(1,0,3,2)
constexpr int kDppQuadSwap2 = 0x4E;      // quad_perm(2,3,0,1)
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int Ctrl>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), Ctrl, 0xf, 0xf, false));
}

__device__ __forceinline__ float row16_sum(float x) {
  x += dpp<kDppQuadSwap1>(x);
  x += dpp<kDppQuadSwap2>(x);
  x += dpp<kDppRowHalfMirror>(x);
  x += dpp<kDppRowMirror>(x);
  return x;
}

__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp<kDppQuadSwap1>(x));
  x = fmaxf(x, dpp<kDppQuadSwap2>(x));
  x = fmaxf(x, dpp<kDppRowHalfMirror>(x));
  x = fmaxf(x, dpp<kDppRowMirror>(x));
  return x;
}

// N independent 16-lane sums advanced in lockstep, so consecutive DPP ops never
// read the register the previous op just wrote (no hazard wait states).
template <int N>
__device__ __forceinline__ void row16_sum_n(float (&x)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) x[i] += dpp<kDppQuadSwap1>(x[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) x[i] += dpp<kDppQuadSwap2>(x[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) x[i] += dpp<kDppRowHalfMirror>(x[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) x[i] += dpp<kDppRowMirror>(x[i]);
}

// Sum over the whole 64-lane wave; all lanes receive the total.
__device__ __forceinline__ float wave_sum(float x) {
  x = row16_sum(x);
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

// s_waitcnt vmcnt(0): block until every outstanding vector-memory load of this
// wave has returned. Used right after loading values that stay live across a
// loop (e.g. the query rows), so the compiler's wait-count tracking does not
// conservatively wait on the loop's own prefetch loads in every iteration.
__device__ __forceinline__ void wait_vmem_loads() {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt=0, expcnt=7, lgkmcnt=15 (gfx9 encoding)
}

// ----------------------------------------------------------------------------
// Direct global -> LDS copies (global_load_lds_dwordx4).
// ----------------------------------------------------------------------------
typedef __attribute__((address_space(3))) uint8_t lds_u8;

// LDS byte address of a __shared__ object (what m0 takes for the copies).
__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_u8*)p));
}

// One 16-byte global -> LDS copy per lane into lds_base + 16 * lane. The compiler
// does not see this write; the kernel orders it with explicit vmcnt waits and
// barriers (the builtin would make every later LDS read wait for all copies).
__device__ __forceinline__ void copy_to_lds(const void* src, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_base), "v"(src)
               : "m0");
}

// One 4-byte global -> LDS copy per lane into lds_base + 4 * lane (same ordering rules).
__device__ __forceinline__ void copy_dword_to_lds(const void* src, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off" ::"s"(lds_base), "v"(src)
               : "m0");
}

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt[3:0] in bits 3:0, vmcnt[5:4] in 15:14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int PER_TILE, int MAX_AHEAD>
__device__ __forceinline__ void wait_tiles_ahead(int ahead) {
  static_assert(MAX_AHEAD <= 4 && PER_TILE * MAX_AHEAD < 64, "vmcnt range");
  if constexpr (MAX_AHEAD >= 4) {
    if (ahead >= 4) {
      wait_vmcnt<PER_TILE * 4>();
      return;
    }
  }
  if constexpr (MAX_AHEAD >= 3) {
    if (ahead >= 3) {
      wait_vmcnt<PER_TILE * 3>();
      return;
    }
  }
  if constexpr (MAX_AHEAD >= 2) {
    if (ahead >= 2) {
      wait_vmcnt<PER_TILE * 2>();
      return;
    }
  }
  if constexpr (MAX_AHEAD >= 1) {
    if (ahead >= 1) {
      wait_vmcnt<PER_TILE>();
      return;
    }
  }
  wait_vmcnt<0>();
}

// 128-bit global loads/stores.
__device__ __forceinline__ uint4 ld128(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}
__device__ __forceinline__ void st128(void* p, const uint4& v) {
  *reinterpret_cast<uint4*>(p) = v;
}

// The decode-batch projection launcher of linear.hip (validation, tiling, split-K). With
// leave_partials the fp32 partials [splits][M][N] stay in `workspace` unreduced and
// *splits_used says how many there are (1: `out` holds the product).
const char* run_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, void* out,
                       int64_t ldo, int64_t M, int64_t N, int64_t K, void* workspace,
                       int64_t workspace_bytes, int32_t cus, int32_t config, int32_t splits,
                       int64_t dtype, bool leave_partials, int* splits_used, hipStream_t s);

}  // namespace mi355x
