// Measured ceilings of MI355X for the two bounds of the attention hot path.
//
// Measurement infrastructure only (bench.py --only ceilings and the default bench
// line's "ceilings" object); it is a separate library (libmi355x_calib.so) and no
// product path loads it. Each kernel isolates one bound:
//   gather: the decode kernels' memory pattern without arithmetic: random 2 KiB K and
//           V rows (page size 1, one row per slot of a permuted pool), every wave
//           reading whole rows with 16-byte loads, grid-stride over the slots;
//   stream: a contiguous read of the same byte count (the HBM streaming rate);
//   mfma:   back-to-back v_mfma_f32_32x32x16_bf16 on operands with random bits (sign,
//           exponent 2^-2..2^1, mantissa), cycling four A operands; MI355X lowers its
//           clock under this load, so the rate is below the nominal dense peak;
//   core:   the prefill kernel's per-tile work on LDS-resident random tiles, 8 waves per
//           workgroup: S^T = K Q^T (16 MFMAs), row max, exp2, P^T packing and row sums,
//           O^T += V^T P^T (16 MFMAs with transposed LDS reads), one barrier per tile;
//   core64: the same work as 4 waves of 64 queries (one wave per SIMD, each K and V
//           fragment feeding two products, half the LDS reads). Both report the shader
//           cycles of every workgroup, so a run gives cycles per tile and the clock the
//           chip held: the two structures take different cycle counts per tile at
//           different clocks for nearly the same time, the signature of a power limit.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef __attribute__((address_space(3))) v4i16_t lds_v4i16;

__device__ __forceinline__ uint32_t mix(uint32_t x) {
  x *= 2654435761u;
  x ^= x >> 15;
  x *= 2246822519u;
  x ^= x >> 13;
  return x;
}
// Two bf16 values with random sign and mantissa, exponent 2^-2 .. 2^1.
__device__ __forceinline__ uint32_t random_bf16x2(uint32_t h) {
  const uint32_t lo = (h & 0x807fu) | ((125u + ((h >> 8) & 3u)) << 7);
  const uint32_t hi = ((h >> 16) & 0x807fu) | ((125u + ((h >> 24) & 3u)) << 7);
  return lo | (hi << 16);
}
__device__ __forceinline__ uint4 random_operand(uint32_t seed) {
  return make_uint4(random_bf16x2(mix(seed)), random_bf16x2(mix(seed + 1)),
                    random_bf16x2(mix(seed + 2)), random_bf16x2(mix(seed + 3)));
}
__device__ __forceinline__ floatx16 mfma(const uint4& a, const uint4& b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// The decode memory pattern without arithmetic: per row (token) the 2 KiB K row and the
// 2 KiB V row at a page-table slot, read into registers. Each wave keeps DEPTH rows
// (DEPTH * 4 KiB, 4 x 16-byte loads per lane per row) in flight per loop trip; the grid is
// `blocks` workgroups of 8 waves. A structure unlike the decode kernel's (register loads,
// many waves per CU, no LDS ring), so its rate bounds the pattern, not one kernel.
template <int DEPTH>
__global__ __launch_bounds__(512) void gather_rows(const uint4* __restrict__ k,
                                                   const uint4* __restrict__ v,
                                                   const int32_t* __restrict__ slots, int rows,
                                                   uint32_t* sink) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int stride = gridDim.x * 8 * DEPTH;
  uint32_t acc = 0;
  for (int r0 = (blockIdx.x * 8 + wave) * DEPTH; r0 < rows; r0 += stride) {
    uint4 x[DEPTH][4];
#pragma unroll
    for (int i = 0; i < DEPTH; ++i) {
      const int64_t s = slots[min(r0 + i, rows - 1)];
      x[i][0] = k[s * 128 + lane];
      x[i][1] = k[s * 128 + 64 + lane];
      x[i][2] = v[s * 128 + lane];
      x[i][3] = v[s * 128 + 64 + lane];
    }
#pragma unroll
    for (int i = 0; i < DEPTH; ++i) acc ^= x[i][0].x ^ x[i][1].y ^ x[i][2].z ^ x[i][3].w;
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

__global__ __launch_bounds__(256) void stream_read(const uint4* __restrict__ p, int64_t n,
                                                   uint32_t* sink) {
  uint32_t acc = 0;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * blockDim.x) {
    const uint4 x = p[i];
    acc ^= x.x ^ x.w;
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

__global__ __launch_bounds__(512) void mfma_random(float* sink, int iters) {
  floatx16 c[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 16; ++i) c[j][i] = 0.f;
  uint4 a[4], b[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t seed = (blockIdx.x * 512 + threadIdx.x) * 16 + j * 4;
    a[j] = random_operand(seed);
    b[j] = random_operand(seed + 0x55555);
  }
  for (int it = 0; it < iters; it += 4)
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) c[j] = mfma(a[(j + u) & 3], b[j], c[j]);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 16; ++i) s += c[j][i];
  if (s == 1234.5f) sink[0] = s;
}

constexpr int kStage = 32768;  // one 64-key K tile + one V tile, bf16, head_dim 128

__global__ __launch_bounds__(512, 1) void attention_core(float* sink, int iters,
                                                         uint64_t* cycles) {
  const uint64_t c_start = __builtin_readcyclecounter();
  __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * kStage];
  const int tid = threadIdx.x, lane = tid & 63, col = lane & 31, half = lane >> 5;
  for (int i = tid; i < 2 * kStage / 4; i += 512)
    reinterpret_cast<uint32_t*>(lds)[i] = random_bf16x2(mix(i + blockIdx.x * 977u));
  __syncthreads();
  uint4 q[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) q[s] = random_operand((blockIdx.x * 512 + tid) * 64 + s * 4);
  const int gq = lane >> 4, p16 = lane & 15;
  const int v_key = 4 * (gq >> 1) + (p16 >> 2);
  const int v_lo = 2 * (gq & 1) + ((p16 >> 1) & 1);
  int v_off[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
    v_off[db] = 16384 + v_key * 256 + ((4 * db + v_lo) ^ (4 * (p16 >> 2))) * 16 + 8 * (p16 & 1);
  floatx16 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.f;
  float m = -1e30f, l = 0.f;
  const float scale = 0.127f;
  const uint32_t ones = pack2(1.f, 1.f);
  for (int t = 0; t < iters; ++t) {
    __syncthreads();
    const uint8_t* sb = lds + (t & 1) * kStage;
    floatx16 s[2];
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[T][r] = 0.f;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
#pragma unroll
      for (int T = 0; T < 2; ++T) {
        const uint4 kf = *reinterpret_cast<const uint4*>(
            sb + (32 * T + col) * 256 + (((2 * kk + half) ^ (col & 15)) * 16));
        s[T] = mfma(kf, q[kk], s[T]);
      }
    float mx = -INFINITY;
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[T][r]);
    const auto sw =
        __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * scale;
    if (__any(mx > m + 8.f)) {
      const float m_new = fmaxf(m, mx);
      const float alpha = __builtin_amdgcn_exp2f(m - m_new);
      m = m_new;
      l *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
    }
    uint4 pb[4];
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        float p[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          p[i] = __builtin_amdgcn_exp2f(fmaf(s[T][8 * hh + i], scale, -m));
        uint4& w = pb[2 * T + hh];
        w = make_uint4(pack2(p[0], p[1]), pack2(p[2], p[3]), pack2(p[4], p[5]), pack2(p[6], p[7]));
        l = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.x),
                                            __builtin_bit_cast(bf16x2_t, ones), l, false);
        l = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.y),
                                            __builtin_bit_cast(bf16x2_t, ones), l, false);
        l = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.z),
                                            __builtin_bit_cast(bf16x2_t, ones), l, false);
        l = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.w),
                                            __builtin_bit_cast(bf16x2_t, ones), l, false);
      }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        lds_u8* vp = (lds_u8*)sb + v_off[db] + 16 * kk * 256;
        const uint2 lo =
            __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)vp));
        const uint2 hi = __builtin_bit_cast(
            uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(vp + 8 * 256)));
        o[db] = mfma(make_uint4(lo.x, lo.y, hi.x, hi.y), pb[kk], o[db]);
      }
  }
  float acc = l;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc += o[db][r];
  if (acc == 1234.5f) sink[0] = acc;
  if (cycles && threadIdx.x == 0) cycles[blockIdx.x] = __builtin_readcyclecounter() - c_start;
}

// The same per-tile work as 4 waves of 64 queries: per wave two 32-query blocks, so each K
// fragment (S^T) and each V^T fragment (O^T) feeds two products.
__global__ __launch_bounds__(256, 1) void attention_core64(float* sink, int iters,
                                                           uint64_t* cycles) {
  const uint64_t c_start = __builtin_readcyclecounter();
  __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * kStage];
  const int tid = threadIdx.x, lane = tid & 63, col = lane & 31, half = lane >> 5;
  for (int i = tid; i < 2 * kStage / 4; i += 256)
    reinterpret_cast<uint32_t*>(lds)[i] = random_bf16x2(mix(i + blockIdx.x * 977u));
  __syncthreads();
  uint4 q[2][8];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int s = 0; s < 8; ++s) q[b][s] = random_operand((blockIdx.x * 512 + 2 * tid + b) * 64 + s * 4);
  const int gq = lane >> 4, p16 = lane & 15;
  const int v_key = 4 * (gq >> 1) + (p16 >> 2);
  const int v_lo = 2 * (gq & 1) + ((p16 >> 1) & 1);
  int v_off[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
    v_off[db] = 16384 + v_key * 256 + ((4 * db + v_lo) ^ (4 * (p16 >> 2))) * 16 + 8 * (p16 & 1);
  floatx16 o[4][2];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[db][b][r] = 0.f;
  float m[2] = {0.f, 0.f}, l[2] = {0.f, 0.f};
  for (int t = 0; t < iters; ++t) {
    __syncthreads();
    const uint8_t* sb = lds + (t & 1) * kStage;
    floatx16 s[2][2];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[0][b][r] = s[1][b][r] = -m[b];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
#pragma unroll
      for (int T = 0; T < 2; ++T) {
        const uint4 kf = *reinterpret_cast<const uint4*>(
            sb + (32 * T + col) * 256 + (((2 * kk + half) ^ (col & 15)) * 16));
#pragma unroll
        for (int b = 0; b < 2; ++b) s[T][b] = mfma(kf, q[b][kk], s[T][b]);
      }
    float mx[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      float v = -INFINITY;
#pragma unroll
      for (int T = 0; T < 2; ++T)
#pragma unroll
        for (int r = 0; r < 16; ++r) v = fmaxf(v, s[T][b][r]);
      const auto sw =
          __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
      mx[b] = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    }
    if (__any(mx[0] > 8.f || mx[1] > 8.f)) {
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const float shift = fmaxf(mx[b], 0.f);
        const float alpha = __builtin_amdgcn_exp2f(-shift);
        m[b] += shift;
        l[b] *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[db][b][r] *= alpha;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          s[0][b][r] -= shift;
          s[1][b][r] -= shift;
        }
      }
    }
    uint4 pb[4][2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      float ls[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int T = 0; T < 2; ++T)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          float p[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            p[i] = __builtin_amdgcn_exp2f(s[T][b][8 * hh + i]);
            ls[i & 3] += p[i];
          }
          pb[2 * T + hh][b] = make_uint4(pack2(p[0], p[1]), pack2(p[2], p[3]),
                                         pack2(p[4], p[5]), pack2(p[6], p[7]));
        }
      l[b] += (ls[0] + ls[1]) + (ls[2] + ls[3]);
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        lds_u8* vp = (lds_u8*)sb + v_off[db] + 16 * kk * 256;
        const uint2 lo =
            __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)vp));
        const uint2 hi = __builtin_bit_cast(
            uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(vp + 8 * 256)));
        const uint4 vf = make_uint4(lo.x, lo.y, hi.x, hi.y);
#pragma unroll
        for (int b = 0; b < 2; ++b) o[db][b] = mfma(vf, pb[kk][b], o[db][b]);
      }
  }
  float acc = l[0] + l[1];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc += o[db][b][r];
  if (acc == 1234.5f) sink[0] = acc;
  if (cycles && threadIdx.x == 0) cycles[blockIdx.x] = __builtin_readcyclecounter() - c_start;
}

}  // namespace

// Each entry point launches one measurement kernel on `stream`; NULL on success.
extern "C" __attribute__((visibility("default"))) const char* mi355x_calib_gather(
    const void* k, const void* v, const int32_t* slots, int32_t rows, void* sink, void* stream) {
  gather_rows<2><<<1024, 512, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint4*>(k), static_cast<const uint4*>(v), slots, rows,
      static_cast<uint32_t*>(sink));
  return hipGetLastError() == hipSuccess ? nullptr : "gather launch failed";
}

// Per-CU load rate of direct global -> LDS copies (the copy the projection and decode kernels
// use): 8 waves per workgroup, each keeping 8 KiB in flight (eight 1 KiB copies per trip, wait
// until 8 remain) on a stream of its own through `bytes` of memory (a multiple of
// blocks * 8 * 1 MiB). With MIX every other copy reads a 1 MiB block at the end of the buffer,
// which stays in L2, so a CU's load queue carries half L2 hits and half HBM misses.
typedef __attribute__((address_space(3))) uint8_t calib_lds_u8;

template <bool MIX>
__global__ __launch_bounds__(512, 1) void load_rate(const uint8_t* __restrict__ buf, int64_t bytes,
                                                    int iters) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[65536];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (iters < 0) lds[threadIdx.x] = 0;  // never taken; the copies' LDS writes are invisible
  const uint32_t base =
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const calib_lds_u8*)lds)) + wave * 8192;
  const int64_t region = bytes / (int64_t(gridDim.x) * 8);
  const int64_t off = (int64_t(blockIdx.x) * 8 + wave) * region;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const int64_t k = (int64_t(it) * 8 + d) * 1024;
      const uint8_t* p = (MIX && (d & 1))
                             ? buf + bytes - (1 << 20) + ((k + wave * 65536) & ((1 << 20) - 1))
                             : buf + off + k % region;
      asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(base + d * 1024),
                   "v"(p + lane * 16)
                   : "m0");
    }
    __builtin_amdgcn_s_waitcnt((8 & 15) | (7 << 4) | (15 << 8));  // vmcnt(8)
  }
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0)
}

extern "C" __attribute__((visibility("default"))) const char* mi355x_calib_load_rate(
    const void* buf, int64_t bytes, int32_t iters, int32_t mix, int32_t blocks, void* stream) {
  if (blocks <= 0 || iters <= 0 || bytes % (int64_t(blocks) * 8 * (1 << 20)))
    return "load rate: bytes must be a multiple of blocks * 8 MiB";
  auto s = static_cast<hipStream_t>(stream);
  auto b = static_cast<const uint8_t*>(buf);
  if (mix)
    load_rate<true><<<blocks, 512, 0, s>>>(b, bytes, iters);
  else
    load_rate<false><<<blocks, 512, 0, s>>>(b, bytes, iters);
  return hipGetLastError() == hipSuccess ? nullptr : "load rate launch failed";
}

// The same gather with DEPTH rows in flight per wave (1, 2, 4 or 8) over `blocks`
// workgroups: the in-flight sweep that shows where the pattern saturates.
extern "C" __attribute__((visibility("default"))) const char* mi355x_calib_gather_depth(
    const void* k, const void* v, const int32_t* slots, int32_t rows, int32_t depth,
    int32_t blocks, void* sink, void* stream) {
  auto s = static_cast<hipStream_t>(stream);
  auto kp = static_cast<const uint4*>(k);
  auto vp = static_cast<const uint4*>(v);
  auto out = static_cast<uint32_t*>(sink);
  switch (depth) {
    case 1: gather_rows<1><<<blocks, 512, 0, s>>>(kp, vp, slots, rows, out); break;
    case 2: gather_rows<2><<<blocks, 512, 0, s>>>(kp, vp, slots, rows, out); break;
    case 4: gather_rows<4><<<blocks, 512, 0, s>>>(kp, vp, slots, rows, out); break;
    case 8: gather_rows<8><<<blocks, 512, 0, s>>>(kp, vp, slots, rows, out); break;
    default: return "gather depth must be 1, 2, 4 or 8";
  }
  return hipGetLastError() == hipSuccess ? nullptr : "gather launch failed";
}

extern "C" __attribute__((visibility("default"))) const char* mi355x_calib_stream(
    const void* p, int64_t bytes, void* sink, void* stream) {
  stream_read<<<4096, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint4*>(p), bytes / 16, static_cast<uint32_t*>(sink));
  return hipGetLastError() == hipSuccess ? nullptr : "stream launch failed";
}

// FLOPs of one launch: blocks * 8 waves * iters * 4 * 32768 (iters a multiple of 4).
extern "C" __attribute__((visibility("default"))) const char* mi355x_calib_mfma(
    int32_t blocks, int32_t iters, void* sink, void* stream) {
  mfma_random<<<blocks, 512, 0, static_cast<hipStream_t>(stream)>>>(static_cast<float*>(sink),
                                                                     iters);
  return hipGetLastError() == hipSuccess ? nullptr : "mfma launch failed";
}

// FLOPs of one launch: blocks * 8 waves * iters * 32 * 32768.
extern "C" __attribute__((visibility("default"))) const char* mi355x_calib_attention_core(
    int32_t blocks, int32_t iters, void* sink, void* stream) {
  attention_core<<<blocks, 512, 0, static_cast<hipStream_t>(stream)>>>(static_cast<float*>(sink),
                                                                       iters, nullptr);
  return hipGetLastError() == hipSuccess ? nullptr : "attention core launch failed";
}

// One launch of the per-tile work with each workgroup's shader cycles written to
// `cycles` (blocks x uint64): variant 0 is the 8-wave x 32-query structure of
// mi355x_calib_attention_core, variant 1 the 4-wave x 64-query one. Both cover 256 query
// rows x 64 keys x 128 dims per workgroup and tile: FLOPs = blocks * iters * 2^23.
extern "C" __attribute__((visibility("default"))) const char* mi355x_calib_attention_core_cycles(
    int32_t blocks, int32_t iters, int32_t variant, void* cycles, void* sink, void* stream) {
  auto s = static_cast<hipStream_t>(stream);
  auto c = static_cast<uint64_t*>(cycles);
  if (variant == 0)
    attention_core<<<blocks, 512, 0, s>>>(static_cast<float*>(sink), iters, c);
  else if (variant == 1)
    attention_core64<<<blocks, 256, 0, s>>>(static_cast<float*>(sink), iters, c);
  else
    return "attention core variant must be 0 or 1";
  return hipGetLastError() == hipSuccess ? nullptr : "attention core launch failed";
}
