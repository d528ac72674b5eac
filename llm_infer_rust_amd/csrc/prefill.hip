// Causal GQA prefill attention (head_dim 128) on gfx950 bf16/fp16 MFMA.
//
// Reference path this replaces:
//   plan: sglang_flashinfer_prepare_prefill  src/models/attention/flashinfer_bridge.cpp:250-310
//         PrefillPlan                        src/models/attention/flashinfer_plan_run.cu:243-274
//   run:  sglang_flashinfer_prefill          flashinfer_bridge.cpp:312-346
//         BatchPrefillWith{Ragged,Paged}KVCacheDispatched  flashinfer_plan_run.cu:277-328
//   math: query i of request r (position prefix_r + i) attends keys j <= prefix_r + i of
//         the same request, softmax(q k^T / sqrt(128)) v; GQA by contiguous head groups
//         (backend.rs:1297-1329, 1455-1498 are the libtorch restatement).
// Mode rule (flashinfer_bridge.cpp:266-273): paged iff some prefix > 0; ragged mode reads
// K/V straight from the (packed) projection rows, paged mode from the KV cache pages.
//
// Kernel design. One workgroup = 4 waves = one (request, query tile, kv head, head group).
// Each wave owns 32 queries of one q head and keeps, per 64-key tile:
//   S^T = K Q^T      (v_mfma_f32_32x32x16: A = K rows from LDS, B = Q^T from registers)
//   O^T += V^T P^T   (A = V^T rows from a transposed LDS copy, B = P^T straight from the
//                     S^T accumulators, no LDS round trip)
// In this transposed form each lane holds one query column, so the online-softmax max/sum
// and the O rescale are per-lane register work plus one cross-half exchange per tile.
// K/V tiles are double-buffered in LDS (one barrier per tile); the g q heads that share
// a kv head are processed by the same workgroup so each K/V byte is fetched once per tile.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <memory>
#include <vector>

#include "common.h"

namespace mi355x {
namespace {

constexpr int kD = 128;
constexpr int kTileK = 64;             // keys per tile
constexpr int kQPerWave = 32;          // queries per wave
constexpr int kKPitch = kD + 8;        // LDS K row pitch (elements): conflict-free b128 reads
constexpr int kVPitch = kTileK + 8;    // LDS V^T row pitch (elements): conflict-free b128 reads
constexpr int kKStage = kTileK * kKPitch;
constexpr int kVStage = kD * kVPitch;
constexpr float kLog2e = 1.4426950408889634f;

// Ablation switches for performance decomposition builds (0 in the library):
//   1: skip the softmax (P = constant), 2: skip the K/V global loads (tiles stay as is).
#ifndef MI355X_PREFILL_ABLATE
#define MI355X_PREFILL_ABLATE 0
#endif

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

template <int DT>
struct Mfma;

template <>
struct Mfma<0> {
  __device__ __forceinline__ static floatx16 run(const uint4& a, const uint4& b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
};

template <>
struct Mfma<1> {
  __device__ __forceinline__ static floatx16 run(const uint4& a, const uint4& b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
};

struct ReqInfo {  // per request, uploaded by the plan
  int32_t q_start, q_len, prefix, page_base;
};

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_sn, q_sh;
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_sn, k_sh, v_sn, v_sh;  // ragged strides; paged: slot stride, head stride
  uint16_t* out;
  int64_t o_sn, o_sh;
  const ReqInfo* reqs;
  const int4* work;  // {request, q_begin, kv_head, head_group}
  const int32_t* indices;
  int32_t num_items, num_q_heads, num_kv_heads, page_size;
  float scale_log2;
};

__device__ __forceinline__ uint32_t lo16x2(uint32_t a, uint32_t b) {  // {a.lo, b.lo}
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t hi16x2(uint32_t a, uint32_t b) {  // {a.hi, b.hi}
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return Elem<DT>::pack2(a, b);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// c + a.lo * b.lo + a.hi * b.hi with fp32 accumulation (v_dot2_f32_bf16 / _f16).
template <int DT>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (DT == 0) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
  } else {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b),
                                  c, false);
  }
}

// NW = waves per workgroup (4 or 8), HPB = q heads per workgroup; each head gets NW/HPB
// waves of 32 queries, so BQ = 32 * NW / HPB queries per workgroup.
template <int DT, int NW, int HPB, bool PAGED>
__global__ __launch_bounds__(64 * NW, NW == 8 ? 1 : 2) void prefill_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t lds_k[2][kKStage];
  __shared__ __attribute__((aligned(16))) uint16_t lds_v[2][kVStage];

  constexpr int kWavesPerHead = NW / HPB;
  constexpr int kBQ = kQPerWave * kWavesPerHead;
  const int tid = threadIdx.x;
  // Wave index as a scalar so every wave-level decision below is a uniform branch.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int col = lane & 31;   // query column / MFMA row index
  const int half = lane >> 5;  // k-half of the MFMA operands

  const int4 w = a.work[blockIdx.x];
  const ReqInfo rq = a.reqs[w.x];
  const int q_begin = w.y;
  const int kvh = w.z;
  const int group = a.num_q_heads / a.num_kv_heads;
  const int qh = kvh * group + w.w * HPB + wave / kWavesPerHead;
  const int wq0 = q_begin + (wave % kWavesPerHead) * kQPerWave;  // wave's first query
  const int kv_len = rq.prefix + rq.q_len;
  const int q_hi = min(q_begin + kBQ, rq.q_len);        // workgroup's query end
  const int keys_needed = min(kv_len, rq.prefix + q_hi);  // causal horizon of the tile
  const int n_tiles = (keys_needed + kTileK - 1) / kTileK;
  const bool wave_active = wq0 < rq.q_len;
  const int wave_last_key = rq.prefix + min(wq0 + kQPerWave, rq.q_len) - 1;

  // Q^T operand: lane holds query (wq0 + col), d = 16 s + 8 half .. +8.
  uint4 qreg[8];
  {
    const int qi = min(wq0 + col, rq.q_len - 1);
    const uint16_t* qp = a.q + static_cast<int64_t>(rq.q_start + qi) * a.q_sn + qh * a.q_sh;
#pragma unroll
    for (int s = 0; s < 8; ++s) qreg[s] = ld128(qp + 16 * s + 8 * half);
    wait_vmem_loads();
  }

  // Global -> register staging of a K/V tile (64 keys x 256 bytes each). A 256-thread
  // slice stages K (row = st/16 + 16 j, 16-byte chunk st%16: 16 lanes read one row) and
  // a 256-thread slice stages V (keys 4 (st%16) + j, chunk st/16: the 16 lanes of an LDS
  // phase then write one contiguous V^T row). With 8 waves the two slices are different
  // waves and share one register set; with 4 waves every thread stages both.
  constexpr bool kSplit = NW == 8;
  const int st = tid & 255;
  const bool does_k = !kSplit || wave < 4;
  const bool does_v = !kSplit || wave >= 4;
  const int k_chunk = st & 15;
  const int k_row = st >> 4;
  const int v_chunk = st >> 4;
  const int v_group = st & 15;
  // Within each 16-key block a V^T row stores the key quads in the order
  // {0-3, 8-11, 4-7, 12-15}: the 8 keys an MFMA lane needs for one k-step
  // (16 st + 4 half + {0..3, 8..11}) are then one contiguous 16-byte read.
  const int v_slot = (v_group & ~3) * 4 + ((v_group & 1) * 8 + (v_group & 2) * 2);
  const uint32_t k_sn = static_cast<uint32_t>(a.k_sn), v_sn = static_cast<uint32_t>(a.v_sn);
  // Ragged rows are addressed from a workgroup-uniform base (the request's first row)
  // with a 32-bit per-lane offset; paged rows from the slot index (64-bit product).
  const uint16_t* k_req = a.k + kvh * a.k_sh + k_chunk * 8 +
                          (PAGED ? 0 : static_cast<int64_t>(rq.q_start) * a.k_sn);
  const uint16_t* v_req = a.v + kvh * a.v_sh + v_chunk * 8 +
                          (PAGED ? 0 : static_cast<int64_t>(rq.q_start) * a.v_sn);
  auto k_key = [&](int t, int j) { return t * kTileK + k_row + 16 * j; };
  auto v_key = [&](int t, int j) { return t * kTileK + 4 * v_group + j; };

  constexpr int kRows = kSplit ? 4 : 8;  // staged 16-byte rows per thread per tile
  uint4 sa[kRows], sb[kRows];            // two register stages (tiles t+1 / t+2)
  // Paged mode: page ids of a tile's rows are loaded one tile before the rows themselves
  // (two alternating sets), so a row load never waits on its index load and the in-order
  // vector-memory counter never has to drain earlier row loads.
  int32_t pa[kRows], pb_[kRows];
  auto load_pages = [&](int t, int32_t (&pg)[kRows]) {
    if constexpr (PAGED) {
      int i = 0;
      if (does_k)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          pg[i++] = a.indices[rq.page_base + min(k_key(t, j), kv_len - 1) / a.page_size];
      if (does_v)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          pg[(kSplit ? 0 : 4) + j] =
              a.indices[rq.page_base + min(v_key(t, j), kv_len - 1) / a.page_size];
    }
  };
  auto row_ptr = [&](int j, int32_t page, const uint16_t* base, uint32_t sn) {
    j = min(j, kv_len - 1);
    if constexpr (PAGED) {
      const uint32_t row = static_cast<uint32_t>(page) * static_cast<uint32_t>(a.page_size) +
                           static_cast<uint32_t>(j % a.page_size);
      return base + static_cast<uint64_t>(row) * sn;
    } else {
      return base + static_cast<uint32_t>(j) * sn;
    }
  };
  auto load_tile = [&](int t, const int32_t (&pg)[kRows], uint4 (&sr)[kRows]) {
    if (MI355X_PREFILL_ABLATE == 2 && t > 0) return;
    if (does_k)
#pragma unroll
      for (int j = 0; j < 4; ++j) sr[j] = ld128(row_ptr(k_key(t, j), pg[j], k_req, k_sn));
    if (does_v)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        sr[(kSplit ? 0 : 4) + j] =
            ld128(row_ptr(v_key(t, j), pg[(kSplit ? 0 : 4) + j], v_req, v_sn));
  };
  auto store_tile = [&](int buf, const uint4 (&sr)[kRows]) {
    if (does_k)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        st128(&lds_k[buf][(k_row + 16 * j) * kKPitch + k_chunk * 8], sr[j]);
    if (does_v) {
      // Transpose 4 keys x 8 dims into 8 rows of V^T (4 keys each, 8 bytes).
      const uint4* vs = sr + (kSplit ? 0 : 4);
      const uint32_t w0[4] = {vs[0].x, vs[0].y, vs[0].z, vs[0].w};
      const uint32_t w1[4] = {vs[1].x, vs[1].y, vs[1].z, vs[1].w};
      const uint32_t w2[4] = {vs[2].x, vs[2].y, vs[2].z, vs[2].w};
      const uint32_t w3[4] = {vs[3].x, vs[3].y, vs[3].z, vs[3].w};
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int d = v_chunk * 8 + 2 * p;
        uint2 even = make_uint2(lo16x2(w0[p], w1[p]), lo16x2(w2[p], w3[p]));
        uint2 odd = make_uint2(hi16x2(w0[p], w1[p]), hi16x2(w2[p], w3[p]));
        *reinterpret_cast<uint2*>(&lds_v[buf][d * kVPitch + v_slot]) = even;
        *reinterpret_cast<uint2*>(&lds_v[buf][(d + 1) * kVPitch + v_slot]) = odd;
      }
    }
  };

  floatx16 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.f;
  float m = -1e30f, l = 0.f;
  const int my_q = wq0 + col;                // query (local index) of this lane
  const int my_horizon = rq.prefix + my_q;   // last visible key of this lane's query

  // Body for one 64-key tile held in LDS buffer `buf`.
  auto compute = [&](int t, int buf) {
    const int k0 = t * kTileK;
    if (wave_active && k0 <= wave_last_key) {
      // S^T for 64 keys: two 32-key blocks.
      floatx16 s[2];
#pragma unroll
      for (int T = 0; T < 2; ++T) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s[T][r] = 0.f;
        const uint16_t* krow = &lds_k[buf][(32 * T + col) * kKPitch + 8 * half];
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
          s[T] = Mfma<DT>::run(*reinterpret_cast<const uint4*>(krow + 16 * kk), qreg[kk], s[T]);
      }
      // Only the diagonal / last tiles need the causal and length mask (uniform branch).
      if (k0 + kTileK - 1 > rq.prefix + wq0 || k0 + kTileK > kv_len) {
        const int limit = min(my_horizon, kv_len - 1) - (k0 + 4 * half);
#pragma unroll
        for (int T = 0; T < 2; ++T)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = 32 * T + (r >> 2) * 8 + (r & 3);
            s[T][r] = key <= limit ? s[T][r] : -INFINITY;
          }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int T = 0; T < 2; ++T)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[T][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32)) * a.scale_log2;  // row max in log2 units
      // Lazy rescale: the reference max m only moves when some row's max exceeds it
      // by more than 8, so p = 2^(s - m) <= 2^8 and O/l are rescaled rarely.
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
      uint4 pb[4];  // P^T operands for the four 16-key k-steps
#pragma unroll
      for (int T = 0; T < 2; ++T)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          float p[8];
#pragma unroll
          for (int i = 0; i < 8; ++i)
            p[i] = MI355X_PREFILL_ABLATE == 1
                       ? s[T][8 * hh + i]
                       : __builtin_amdgcn_exp2f(fmaf(s[T][8 * hh + i], a.scale_log2, -m));
          pb[2 * T + hh] = make_uint4(pack2<DT>(p[0], p[1]), pack2<DT>(p[2], p[3]),
                                      pack2<DT>(p[4], p[5]), pack2<DT>(p[6], p[7]));
        }
      // Row sum of the rounded P the PV product uses (v_dot2 against {1, 1}).
      const uint32_t ones = pack2<DT>(1.f, 1.f);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        l = dot2<DT>(pb[kk].x, ones, l);
        l = dot2<DT>(pb[kk].y, ones, l);
        l = dot2<DT>(pb[kk].z, ones, l);
        l = dot2<DT>(pb[kk].w, ones, l);
      }
      // O^T += V^T P^T; k-step kk covers keys 16 kk + 4 half + {0..3, 8..11}, the same
      // order the S^T accumulators hold.
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const uint16_t* vrow = &lds_v[buf][(32 * db + col) * kVPitch + 8 * half];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          o[db] = Mfma<DT>::run(*reinterpret_cast<const uint4*>(vrow + 16 * kk), pb[kk], o[db]);
      }
    }
  };

  // Two LDS buffers and two register stages: while tile t is consumed, tile t+1
  // waits in registers (stored to LDS after the compute) and tile t+2 is in flight.
  // Page ids run one tile further ahead (pa: even tiles, pb_: odd tiles).
  load_pages(0, pa);
  load_pages(1, pb_);
  if (n_tiles > 0) {
    load_tile(0, pa, sa);
    store_tile(0, sa);
  }
  load_pages(2, pa);
  if (n_tiles > 1) load_tile(1, pb_, sb);
  load_pages(3, pb_);
  __syncthreads();
  for (int t = 0; t < n_tiles; t += 2) {
    if (t + 2 < n_tiles) {
      load_tile(t + 2, pa, sa);
      load_pages(t + 4, pa);
    }
    compute(t, 0);
    if (t + 1 < n_tiles) store_tile(1, sb);
    __syncthreads();
    if (t + 1 >= n_tiles) break;
    if (t + 3 < n_tiles) {
      load_tile(t + 3, pb_, sb);
      load_pages(t + 5, pb_);
    }
    compute(t + 1, 1);
    if (t + 2 < n_tiles) store_tile(0, sa);
    __syncthreads();
  }

  if (!wave_active || my_q >= rq.q_len) return;
  const float inv = 1.f / (l + __shfl_xor(l, 32));
  uint16_t* op = a.out + static_cast<int64_t>(rq.q_start + my_q) * a.o_sn + qh * a.o_sh;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d = 32 * db + 8 * g4 + 4 * half;
      const uint2 val = make_uint2(pack2<DT>(o[db][4 * g4] * inv, o[db][4 * g4 + 1] * inv),
                                   pack2<DT>(o[db][4 * g4 + 2] * inv, o[db][4 * g4 + 3] * inv));
      *reinterpret_cast<uint2*>(op + d) = val;
    }
}

__global__ __launch_bounds__(256) void pack_prefill_pages(const int32_t* __restrict__ table,
                                                          const int32_t* __restrict__ indptr,
                                                          int32_t* __restrict__ indices,
                                                          int64_t stride) {
  const int row = blockIdx.x;
  const int begin = indptr[row];
  const int pages = indptr[row + 1] - begin;
  const int32_t* src = table + row * stride;
  for (int c = threadIdx.x; c < pages; c += blockDim.x) indices[begin + c] = src[c];
}

struct Buffer {
  void* ptr = nullptr;
  size_t capacity = 0;
  bool pinned = false;
  hipError_t reserve(size_t bytes, uint64_t& allocations) {
    if (bytes <= capacity) return hipSuccess;
    size_t grown = std::max(bytes, capacity ? capacity * 2 : size_t(65536));
    void* fresh = nullptr;
    hipError_t st = pinned ? hipHostMalloc(&fresh, grown, hipHostMallocDefault)
                           : hipMalloc(&fresh, grown);
    if (st != hipSuccess) return st;
    release();
    ptr = fresh;
    capacity = grown;
    ++allocations;
    return hipSuccess;
  }
  void release() {
    if (ptr) {
      if (pinned)
        (void)hipHostFree(ptr);
      else
        (void)hipFree(ptr);
    }
    ptr = nullptr;
    capacity = 0;
  }
  ~Buffer() { release(); }
};

// Waves per prefill workgroup: 8 (one workgroup per CU, 2 waves per SIMD, twice the
// queries per K/V tile) for paged plans, whose long cached prefixes make K/V staging
// the cost to amortise; 4 (two workgroups per CU, more workgroups) for ragged plans,
// whose causal tail favours finer work items. Measured on MI355X at configs 3 and 4.
// MI355X_PREFILL_WAVES=4|8 overrides both (tuning knob, read once).
int prefill_waves(bool paged) {
  static const int forced = [] {
    const char* env = std::getenv("MI355X_PREFILL_WAVES");
    const int v = env ? std::atoi(env) : 0;
    return (v == 4 || v == 8) ? v : 0;
  }();
  return forced ? forced : (paged ? 8 : 4);
}

int heads_per_block(int64_t group, int waves) {
  return static_cast<int>(std::min<int64_t>(group, waves));
}

}  // namespace

struct PrefillPlan {
  int device = -1;
  int64_t num_q_heads = 0, num_kv_heads = 0, page_size = 0, dtype = 0;
  int64_t batch = 0, total_q = 0, num_items = 0, total_pages = 0;
  bool paged = false;
  int waves = 8;  // waves per workgroup the work list was built for
  // Device int32 workspace: [req info 4*B][work 4*items][kv_indptr B+1][last_len B]
  int64_t o_work = 0, o_indptr = 0, o_last = 0;
  Buffer ints, indices, staging;
  hipEvent_t upload_done = nullptr;
  uint64_t allocations = 0;
  PrefillPlan() { staging.pinned = true; }
  ~PrefillPlan() {
    if (upload_done) {
      (void)hipEventSynchronize(upload_done);
      (void)hipEventDestroy(upload_done);
    }
  }
};

}  // namespace mi355x

using namespace mi355x;

// Host-only: the work list a prefill plan launches. Returns the item count (or -1).
extern "C" int64_t mi355x_prefill_schedule(const int32_t* q_host, const int32_t* prefix_host,
                                           int64_t batch, int64_t num_q_heads,
                                           int64_t num_kv_heads, int32_t* work,
                                           int64_t capacity) {
  if (!q_host || !prefix_host || batch <= 0 || num_kv_heads <= 0 ||
      num_q_heads % num_kv_heads != 0)
    return -1;
  const int64_t group = num_q_heads / num_kv_heads;
  bool paged = false;
  for (int64_t r = 0; r < batch; ++r) paged |= prefix_host[r] > 0;
  const int waves = prefill_waves(paged);
  const int hpb = heads_per_block(group, waves);
  if (group % hpb) return -1;
  const int bq = kQPerWave * (waves / hpb);
  struct Item {
    int64_t cost;
    int32_t r, q0, kvh, hg;
  };
  std::vector<Item> items;
  for (int64_t r = 0; r < batch; ++r) {
    const int64_t q_len = q_host[r + 1] - q_host[r];
    if (q_len <= 0 || prefix_host[r] < 0) return -1;
    for (int64_t q0 = 0; q0 < q_len; q0 += bq) {
      const int64_t horizon = prefix_host[r] + std::min<int64_t>(q0 + bq, q_len);
      const int64_t cost = (horizon + kTileK - 1) / kTileK;
      for (int64_t h = 0; h < num_kv_heads; ++h)
        for (int64_t g = 0; g < group / hpb; ++g)
          items.push_back({cost, static_cast<int32_t>(r), static_cast<int32_t>(q0),
                           static_cast<int32_t>(h), static_cast<int32_t>(g)});
    }
  }
  // Longest first: the heavy causal tail starts early and the short tiles fill the gaps.
  std::stable_sort(items.begin(), items.end(),
                   [](const Item& x, const Item& y) { return x.cost > y.cost; });
  const int64_t n = static_cast<int64_t>(items.size());
  if (work) {
    if (n > capacity) return -1;
    for (int64_t i = 0; i < n; ++i) {
      work[4 * i] = items[i].r;
      work[4 * i + 1] = items[i].q0;
      work[4 * i + 2] = items[i].kvh;
      work[4 * i + 3] = items[i].hg;
    }
  }
  return n;
}

extern "C" void* mi355x_prefill_prepare(void* existing, const int32_t* q_indptr,
                                        const int32_t* block_table, int64_t batch,
                                        int64_t columns, int64_t table_stride,
                                        const int32_t* q_host, const int32_t* prefix_host,
                                        int64_t num_q_heads, int64_t num_kv_heads,
                                        int64_t page_size, int64_t dtype, void* stream) {
  auto s = static_cast<hipStream_t>(stream);
  std::unique_ptr<PrefillPlan> created;
  auto* plan = static_cast<PrefillPlan*>(existing);
  try {
    if (!q_indptr || !q_host || !prefix_host || batch <= 0 || page_size <= 0 ||
        (dtype != 0 && dtype != 1) || num_q_heads <= 0 || num_kv_heads <= 0 ||
        num_q_heads % num_kv_heads != 0) {
      set_error("invalid prefill metadata");
      return nullptr;
    }
    const int64_t group = num_q_heads / num_kv_heads;
    if (group != 1 && group != 2 && group != 4 && group != 8) {
      set_error("prefill supports 1, 2, 4 or 8 query heads per kv head");
      return nullptr;
    }
    bool paged = false;
    for (int64_t i = 0; i < batch; ++i) {
      if (prefix_host[i] < 0 || q_host[i + 1] <= q_host[i] || q_host[0] != 0) {
        set_error("invalid prefill lengths");
        return nullptr;
      }
      if (block_table &&
          (int64_t(prefix_host[i]) + q_host[i + 1] - q_host[i] + page_size - 1) / page_size >
              columns) {
        set_error("prefill block table is too small");
        return nullptr;
      }
      paged |= prefix_host[i] > 0;
    }
    if (paged && (!block_table || columns <= 0 || table_stride < columns)) {
      set_error("paged prefill requires a block table");
      return nullptr;
    }
    int device = 0;
    hipError_t st = hipGetDevice(&device);
    if (st != hipSuccess) {
      hip_error(st, "hipGetDevice");
      return nullptr;
    }
    if (plan && (plan->device != device || plan->num_q_heads != num_q_heads ||
                 plan->num_kv_heads != num_kv_heads || plan->page_size != page_size ||
                 plan->dtype != dtype)) {
      set_error("prefill geometry changed");
      return nullptr;
    }
    if (!plan) {
      created = std::make_unique<PrefillPlan>();
      plan = created.get();
      plan->device = device;
      plan->num_q_heads = num_q_heads;
      plan->num_kv_heads = num_kv_heads;
      plan->page_size = page_size;
      plan->dtype = dtype;
      st = hipEventCreateWithFlags(&plan->upload_done, hipEventDisableTiming);
      if (st != hipSuccess) {
        hip_error(st, "hipEventCreate");
        return nullptr;
      }
    }
    const int64_t n_items =
        mi355x_prefill_schedule(q_host, prefix_host, batch, num_q_heads, num_kv_heads, nullptr, 0);
    if (n_items <= 0 || n_items > std::numeric_limits<int32_t>::max()) {
      set_error("prefill work list is empty or too large");
      return nullptr;
    }
    const int64_t o_work = 4 * batch;
    const int64_t o_indptr = o_work + 4 * n_items;
    const int64_t o_last = o_indptr + batch + 1;
    const int64_t total_ints = o_last + batch;
    st = hipEventSynchronize(plan->upload_done);
    if (st != hipSuccess) {
      hip_error(st, "prefill upload fence");
      return nullptr;
    }
    if ((st = plan->ints.reserve(total_ints * 4, plan->allocations)) != hipSuccess ||
        (st = plan->staging.reserve(total_ints * 4, plan->allocations)) != hipSuccess) {
      hip_error(st, "prefill workspace allocation");
      return nullptr;
    }
    int32_t* host = static_cast<int32_t*>(plan->staging.ptr);
    int64_t total_pages = 0;
    host[o_indptr] = 0;
    for (int64_t r = 0; r < batch; ++r) {
      const int64_t q_len = q_host[r + 1] - q_host[r];
      const int64_t kv_len = prefix_host[r] + q_len;
      host[4 * r] = q_host[r];
      host[4 * r + 1] = static_cast<int32_t>(q_len);
      host[4 * r + 2] = prefix_host[r];
      host[4 * r + 3] = static_cast<int32_t>(total_pages);
      if (paged) {
        total_pages += (kv_len + page_size - 1) / page_size;
        if (total_pages > std::numeric_limits<int32_t>::max()) {
          set_error("prefill page indptr overflow");
          return nullptr;
        }
        host[o_indptr + r + 1] = static_cast<int32_t>(total_pages);
        host[o_last + r] = static_cast<int32_t>((kv_len - 1) % page_size + 1);
      } else {
        host[o_indptr + r + 1] = q_host[r + 1];  // ragged: kv indptr is the q indptr
        host[o_last + r] = 0;
      }
    }
    mi355x_prefill_schedule(q_host, prefix_host, batch, num_q_heads, num_kv_heads,
                            host + o_work, n_items);
    st = hipMemcpyAsync(plan->ints.ptr, host, total_ints * 4, hipMemcpyHostToDevice, s);
    if (st != hipSuccess) {
      hip_error(st, "prefill metadata upload");
      return nullptr;
    }
    if (paged) {
      if ((st = plan->indices.reserve(std::max<int64_t>(total_pages, 1) * 4, plan->allocations)) !=
          hipSuccess) {
        hip_error(st, "prefill index allocation");
        return nullptr;
      }
      pack_prefill_pages<<<dim3(static_cast<uint32_t>(batch)), dim3(256), 0, s>>>(
          block_table, static_cast<const int32_t*>(plan->ints.ptr) + o_indptr,
          static_cast<int32_t*>(plan->indices.ptr), table_stride);
      if (launch_status("pack_prefill_pages")) return nullptr;
    }
    st = hipEventRecord(plan->upload_done, s);
    if (st != hipSuccess) {
      hip_error(st, "prefill upload event");
      return nullptr;
    }
    plan->batch = batch;
    plan->total_q = q_host[batch];
    plan->num_items = n_items;
    plan->total_pages = total_pages;
    plan->paged = paged;
    plan->waves = prefill_waves(paged);
    plan->o_work = o_work;
    plan->o_indptr = o_indptr;
    plan->o_last = o_last;
    created.release();
    return plan;
  } catch (const std::exception& e) {
    set_error(e.what());
    return nullptr;
  }
}

extern "C" void mi355x_prefill_plan_drop(void* plan) { delete static_cast<PrefillPlan*>(plan); }

extern "C" uint64_t mi355x_prefill_workspace_allocations(const void* plan) {
  return plan ? static_cast<const PrefillPlan*>(plan)->allocations : 0;
}

// Plan facts: out6 = {batch, total_q, paged, num_items, total_pages, 0}.
extern "C" const char* mi355x_prefill_plan_info(const void* plan, int64_t* out6) {
  if (!plan || !out6) return set_error("mi355x_prefill_plan_info: null argument");
  const auto* p = static_cast<const PrefillPlan*>(plan);
  out6[0] = p->batch;
  out6[1] = p->total_q;
  out6[2] = p->paged ? 1 : 0;
  out6[3] = p->num_items;
  out6[4] = p->total_pages;
  out6[5] = 0;
  return nullptr;
}

extern "C" const char* mi355x_prefill_plan_read(const void* plan, int32_t* kv_indptr,
                                                int32_t* indices, int32_t* last_len,
                                                void* stream) {
  if (!plan) return set_error("mi355x_prefill_plan_read: null plan");
  const auto* p = static_cast<const PrefillPlan*>(plan);
  auto s = static_cast<hipStream_t>(stream);
  const int32_t* ints = static_cast<const int32_t*>(p->ints.ptr);
  hipError_t st = hipSuccess;
  auto copy = [&](void* dst, const void* src, size_t bytes) {
    if (dst && st == hipSuccess && bytes)
      st = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s);
  };
  copy(kv_indptr, ints + p->o_indptr, (p->batch + 1) * 4);
  if (p->paged) {
    copy(indices, p->indices.ptr, p->total_pages * 4);
    copy(last_len, ints + p->o_last, p->batch * 4);
  }
  if (st == hipSuccess) st = hipStreamSynchronize(s);
  return st == hipSuccess ? nullptr : hip_error(st, "mi355x_prefill_plan_read");
}

namespace mi355x {
namespace {
template <int DT, int NW, int HPB>
void launch_prefill(const PrefillArgs& a, bool paged, hipStream_t s) {
  const dim3 grid(static_cast<uint32_t>(a.num_items)), block(64 * NW);
  if (paged)
    prefill_kernel<DT, NW, HPB, true><<<grid, block, 0, s>>>(a);
  else
    prefill_kernel<DT, NW, HPB, false><<<grid, block, 0, s>>>(a);
}
template <int DT>
void launch_dt(const PrefillArgs& a, int waves, int hpb, bool paged, hipStream_t s) {
  if (waves == 8) {
    if (hpb == 1) launch_prefill<DT, 8, 1>(a, paged, s);
    else if (hpb == 2) launch_prefill<DT, 8, 2>(a, paged, s);
    else if (hpb == 4) launch_prefill<DT, 8, 4>(a, paged, s);
    else launch_prefill<DT, 8, 8>(a, paged, s);
  } else {
    if (hpb == 1) launch_prefill<DT, 4, 1>(a, paged, s);
    else if (hpb == 2) launch_prefill<DT, 4, 2>(a, paged, s);
    else launch_prefill<DT, 4, 4>(a, paged, s);
  }
}
}  // namespace
}  // namespace mi355x

extern "C" const char* mi355x_prefill_run(const void* plan_ptr, const void* q, int64_t q_sn,
                                          int64_t q_sh, const void* k, int64_t k_sn,
                                          int64_t k_sh, const void* v, int64_t v_sn,
                                          int64_t v_sh, void* out, int64_t o_sn, int64_t o_sh,
                                          int64_t total_q, int64_t num_q_heads,
                                          int64_t num_kv_heads, int64_t page_size, int64_t dtype,
                                          void* stream) {
  if (!plan_ptr) return set_error("prefill was not prepared");
  const auto& p = *static_cast<const PrefillPlan*>(plan_ptr);
  if (!q || !k || !v || !out) return set_error("mi355x_prefill_run: null pointer");
  if (total_q != p.total_q || num_q_heads != p.num_q_heads || num_kv_heads != p.num_kv_heads ||
      page_size != p.page_size || dtype != p.dtype)
    return set_error("prefill shape mismatch");
  if (q_sn % 8 || q_sh % 8 || k_sn % 8 || k_sh % 8 || v_sn % 8 || v_sh % 8 || o_sn % 8 ||
      o_sh % 8 || !aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(out, 16))
    return set_error("prefill requires 16-byte aligned rows");
  PrefillArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.q_sn = q_sn;
  a.q_sh = q_sh;
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.k_sn = k_sn;
  a.k_sh = k_sh;
  a.v_sn = v_sn;
  a.v_sh = v_sh;
  a.out = static_cast<uint16_t*>(out);
  a.o_sn = o_sn;
  a.o_sh = o_sh;
  const int32_t* ints = static_cast<const int32_t*>(p.ints.ptr);
  a.reqs = reinterpret_cast<const ReqInfo*>(ints);
  a.work = reinterpret_cast<const int4*>(ints + p.o_work);
  a.indices = static_cast<const int32_t*>(p.indices.ptr);
  a.num_items = static_cast<int32_t>(p.num_items);
  a.num_q_heads = static_cast<int32_t>(num_q_heads);
  a.num_kv_heads = static_cast<int32_t>(num_kv_heads);
  a.page_size = static_cast<int32_t>(p.paged ? page_size : 1);
  a.scale_log2 = (1.0f / std::sqrt(static_cast<float>(kD))) * kLog2e;
  const int waves = p.waves;
  const int hpb = heads_per_block(num_q_heads / num_kv_heads, waves);
  auto s = static_cast<hipStream_t>(stream);
  if (dtype == 0)
    launch_dt<0>(a, waves, hpb, p.paged, s);
  else
    launch_dt<1>(a, waves, hpb, p.paged, s);
  return launch_status("prefill_kernel");
}
