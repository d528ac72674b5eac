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
// Kernel design. One workgroup = 8 waves (two per SIMD) = one (request, query tile, kv
// head, head group). Each wave owns 32 queries of one q head and keeps, per 64-key tile:
//   S^T = K Q^T      (v_mfma_f32_32x32x16: A = K rows from LDS, B = Q^T from registers)
//   O^T += V^T P^T   (A = V^T read transposed from the row-major V tile with
//                     ds_read_b64_tr_b16, B = P^T straight from the S^T accumulators)
// In this transposed form each lane holds one query column, so the online-softmax max/sum
// and the O rescale are per-lane register work plus one cross-half exchange per tile.
// K/V tiles stream through a 4-deep LDS ring filled by direct global -> LDS copies (one
// barrier per tile); the g q heads that share a kv head are processed by the same
// workgroup so each K/V byte is fetched once per tile.
// Split-KV: when a batch has too few items to fill the device (a long prefix under few
// queries), the plan cuts items into chunks of key tiles; each chunk writes a normalised
// fp32 partial and its log2-sum-exp, and prefill_merge_kernel combines them.
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
constexpr int kTileK = 64;                    // keys per tile
constexpr int kQPerWave = 32;                 // queries per wave
constexpr int kWaves = 8;                     // waves per workgroup
constexpr int kStages = 4;                    // LDS ring depth (tiles)
constexpr int kTileBytes = kTileK * kD * 2;   // 16 KB per K or V tile
constexpr int kStageBytes = 2 * kTileBytes;   // K + V
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMaxKvLen = 1 << 22;            // div_small is exact below this

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
  const int4* work;    // {request, q_begin, kv_head, head_group}
  const int4* ranges;  // per item {first tile, end tile, partial record or -1, 0}
  float* part_o;       // split items: [record][8 slots][32 queries][128] normalised O
  float* part_lse;     // split items: [record][8 slots][32 queries] log2-sum-exp
  const int32_t* indices;
  int32_t num_items, num_q_heads, num_kv_heads, page_size;
  float scale_log2;
};

template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return Elem<DT>::pack2(a, b);
}


// ---------------------------------------------------------------------------
// Tile staging. K and V tiles are copied global -> LDS by the
// load engine (global_load_lds_dwordx4: each lane's 16 bytes land at
// LDS base + 16 * lane), so staging takes no registers and no LDS-store
// instructions, and up to STAGES-1 tiles are in flight. Both tiles keep the
// natural [key][d] layout with 16-byte chunks XOR-swizzled per row:
//   K: chunk c of key r sits at position c ^ (r & 15)  -> the S^T operand reads
//      (one 16-byte chunk of 32 consecutive keys) touch every bank once per 16 lanes;
//   V: chunk c of key r sits at position c ^ 4 (r & 3) -> the transposed reads
//      (ds_read_b64_tr_b16, 4 keys x 64 bytes per 16 lanes) are conflict-free.
// The V^T operand of O^T += V^T P^T comes straight from the row-major tile through
// ds_read_b64_tr_b16: within 16 lanes it returns lane i the 4 elements
// {M[4j + i/4][i%4]}_j of the 16 x 4 block M whose row p the lane p addressed.
// ---------------------------------------------------------------------------

typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16_t lds_v4i16;

// q = x / d, r = x % d for 0 <= x < 2^22 and 1 <= d, via a float reciprocal and one
// correction step each way.
__device__ __forceinline__ int div_small(int x, int d, float inv, int& r) {
  int q = static_cast<int>(static_cast<float>(x) * inv);
  r = x - q * d;
  if (r >= d) {
    ++q;
    r -= d;
  }
  if (r < 0) {
    --q;
    r += d;
  }
  return q;
}

// NW waves per workgroup: 8 (one workgroup per CU, a 4-stage ring) or 4 (two workgroups
// per CU, a 2-stage ring each, so one workgroup's prologue, epilogue and barriers overlap
// the other's tiles).
template <int DT, int HPB, bool PAGED, int NW>
__global__ __launch_bounds__(64 * NW, NW == 8 ? 1 : 2) void prefill_kernel(PrefillArgs a) {
  constexpr int STAGES = NW == 8 ? kStages : 2;
  constexpr int kAhead = STAGES - 1;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[STAGES * kStageBytes];

  constexpr int kWavesPerHead = NW / HPB;
  constexpr int kBQ = kQPerWave * kWavesPerHead;
  constexpr int kGroupsPerWave = 16 / NW;         // 4-row groups of each tile this wave copies
  constexpr int kCopiesPerTile = 2 * kGroupsPerWave;  // K + V copies per wave per tile
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int col = lane & 31;
  const int half = lane >> 5;

  // The tiles are written only by the load engine, which the compiler does not see;
  // one (never taken) visible store keeps it from treating the array as undefined.
  if (a.num_items < 0) lds[tid] = 0;

  const int4 w = a.work[blockIdx.x];
  if (w.x < 0) return;  // padding slot of the XCD-ordered work list
  const int4 range = a.ranges[blockIdx.x];
  const ReqInfo rq = a.reqs[w.x];
  const int q_begin = w.y;
  const int kvh = w.z;
  const int group = a.num_q_heads / a.num_kv_heads;
  // In an 8-wave workgroup waves w and w + 4 share a SIMD. The upper four waves take
  // their (head, query slot) in mirrored order, so each SIMD pairs an early query slot
  // with a late one and the causal tiles near the diagonal, where late slots still work
  // and early ones are done, are spread over all four SIMDs. (A 4-wave workgroup has one
  // wave per SIMD; its partner is a wave of the CU's other workgroup.)
  static_assert(NW == 8 || NW == 4, "8 or 4 waves per workgroup");
  const int slot_id = NW == 8 && wave >= 4 ? 11 - wave : wave;
  const int qh = kvh * group + w.w * HPB + slot_id / kWavesPerHead;
  const int wq0 = q_begin + (slot_id % kWavesPerHead) * kQPerWave;
  const int kv_len = rq.prefix + rq.q_len;
  const int q_hi = min(q_begin + kBQ, rq.q_len);
  const int keys_needed = min(kv_len, rq.prefix + q_hi);
  const int n_tiles = (keys_needed + kTileK - 1) / kTileK;
  // This item's key tiles: all of them, or one chunk of a split item, whose normalised
  // partial result goes to a partial record for the merge launch.
  const int t_begin = range.x;
  const int nt = min(range.y, n_tiles) - t_begin;
  const int pslot = range.z;
  const bool wave_active = wq0 < rq.q_len;
  const int wave_last_key = rq.prefix + min(wq0 + kQPerWave, rq.q_len) - 1;

  uint4 qreg[8];
  {
    const int qi = min(wq0 + col, rq.q_len - 1);
    const uint16_t* qp = a.q + static_cast<int64_t>(rq.q_start + qi) * a.q_sn + qh * a.q_sh;
#pragma unroll
    for (int s = 0; s < 8; ++s) qreg[s] = ld128(qp + 16 * s + 8 * half);
    wait_vmem_loads();
    // The query rows enter the matrix cores as they are: the softmax scale (and log2 e) is
    // applied to the fp32 scores. Folding it into the rows would round q * scale to the
    // input type, a score error that grows with the size of the products q_d k_d.
    // Keep the rows in registers behind an empty asm the compiler cannot look through, so
    // they are never reloaded inside the tile loop (at 250+ VGPRs that would be the cheap
    // way out for the register allocator).
#pragma unroll
    for (int s = 0; s < 8; ++s)
      asm volatile("" : "+v"(qreg[s].x), "+v"(qreg[s].y), "+v"(qreg[s].z), "+v"(qreg[s].w));
  }

  const uint32_t lds_base = lds_address(lds);

  // Copy side: this wave copies row groups g = wave * kGroupsPerWave + j of the K and
  // the V tile; lane -> row 4 g + lane / 16, LDS chunk position lane % 16.
  const int row_in_group = lane >> 4;
  const int pos = lane & 15;
  const uint16_t* k_req = a.k + kvh * a.k_sh + (PAGED ? 0 : static_cast<int64_t>(rq.q_start) * a.k_sn);
  const uint16_t* v_req = a.v + kvh * a.v_sh + (PAGED ? 0 : static_cast<int64_t>(rq.q_start) * a.v_sn);
  const float inv_page = 1.0f / static_cast<float>(a.page_size);

  // Copy one tile (this wave's 4-row groups of K and V) into `stage`. Paged mode: the 4
  // rows of a group span at most 4 consecutive pages, starting at the page of the
  // group's first (clamped) key; their ids are read with one uniform load from the
  // constant address space (the words are read-only here), which becomes a scalar load
  // counted on lgkmcnt and so never waits on the tile copies counted by vmcnt.
  auto issue_general = [&](int t, int stage) {
    const uint32_t sbase = lds_base + stage * kStageBytes;
#pragma unroll
    for (int j = 0; j < kGroupsPerWave; ++j) {
      const int g = wave * kGroupsPerWave + j;
      const int row = 4 * g + row_in_group;
      // Keys past the end are clamped to the last key (finite data, masked later).
      const int key = min(t * kTileK + row, kv_len - 1);
      int64_t slot;
      if constexpr (PAGED) {
        const int key0 =
            __builtin_amdgcn_readfirstlane(min(t * kTileK + 4 * g, (kv_len - 1) & ~3));
        int r0;
        const int p0 = __builtin_amdgcn_readfirstlane(div_small(key0, a.page_size, inv_page, r0));
        const __attribute__((address_space(4))) int32_t* pw =
            (const __attribute__((address_space(4))) int32_t*)(a.indices) + rq.page_base + p0;
        const int i0 = pw[0], i1 = pw[1], i2 = pw[2], i3 = pw[3];
        int off;
        const int sel = div_small(key, a.page_size, inv_page, off) - p0;
        const int page = sel == 0 ? i0 : sel == 1 ? i1 : sel == 2 ? i2 : i3;
        slot = static_cast<int64_t>(page) * a.page_size + off;
      } else {
        slot = key;
      }
      const int kc = pos ^ (row & 15);
      const int vc = pos ^ (4 * (row & 3));
      copy_to_lds(k_req + slot * a.k_sn + kc * 8, sbase + g * 1024);
      copy_to_lds(v_req + slot * a.v_sn + vc * 8, sbase + kTileBytes + g * 1024);
    }
  };

  // Every tile but an item's last lies wholly inside the keys, so no clamping is needed
  // and the per-lane part of each copy address is fixed for the whole loop: row r of
  // tile t sits at lane_k + (key or slot of its group's first row) * stride. Ragged
  // mode: key t * 64 + 4 g. Paged mode with a page size of 4..64 that divides 64 (the
  // serving sizes): the 4 rows of a group lie in one page, so the group needs one
  // page id (page t * 64 / P + 4 g / P of the request) and one uniform multiply.
  const bool fast_pages = !PAGED || (a.page_size >= 4 && a.page_size <= kTileK &&
                                     kTileK % a.page_size == 0);
  const uint16_t* lane_k[kGroupsPerWave];
  const uint16_t* lane_v[kGroupsPerWave];
#pragma unroll
  for (int j = 0; j < kGroupsPerWave; ++j) {
    const int g = wave * kGroupsPerWave + j;
    const int row = 4 * g + row_in_group;
    const int kc = pos ^ (row & 15);
    const int vc = pos ^ (4 * (row & 3));
    lane_k[j] = k_req + static_cast<int64_t>(row_in_group) * a.k_sn + kc * 8;
    lane_v[j] = v_req + static_cast<int64_t>(row_in_group) * a.v_sn + vc * 8;
  }
  const int pages_per_tile = PAGED && fast_pages ? kTileK / a.page_size : 0;
  const int last_page = PAGED ? (kv_len - 1) / a.page_size : 0;
  // Paged fast path: the page id of each of this wave's row groups, for the tile
  // issued next. They are loaded one loop iteration before their copies are issued,
  // so the scalar loads' latency is hidden behind a tile of compute instead of
  // stalling the copy issue right after the barrier.
  int ids[kGroupsPerWave];
  auto load_ids = [&](int t) {
#pragma unroll
    for (int j = 0; j < kGroupsPerWave; ++j) {
      const int g = wave * kGroupsPerWave + j;
      const int p = min(t * pages_per_tile + (4 * g) / a.page_size, last_page);
      ids[j] = *((const __attribute__((address_space(4))) int32_t*)(a.indices) + rq.page_base + p);
    }
  };
  auto issue_fast = [&](int t, int stage) {
    const uint32_t sbase = lds_base + stage * kStageBytes;
#pragma unroll
    for (int j = 0; j < kGroupsPerWave; ++j) {
      const int g = wave * kGroupsPerWave + j;
      int64_t first;  // key (ragged) or slot (paged) of the group's first row
      if constexpr (PAGED) {
        first = static_cast<int64_t>(ids[j]) * a.page_size + (4 * g) % a.page_size;
      } else {
        first = t * kTileK + 4 * g;
      }
      copy_to_lds(lane_k[j] + first * a.k_sn, sbase + g * 1024);
      copy_to_lds(lane_v[j] + first * a.v_sn, sbase + kTileBytes + g * 1024);
    }
  };
  // Issues tile t; in paged mode the ids must hold tile t's page ids, and on return
  // they hold tile t + 1's.
  auto issue = [&](int t, int stage) {
    if (fast_pages && t + 1 < n_tiles)
      issue_fast(t, stage);
    else
      issue_general(t, stage);
    if constexpr (PAGED) {
      if (fast_pages) load_ids(t + 1);
    }
  };

  // Read side offsets (bytes within a stage).
  // K operand: key 32 T + col, chunk 2 kk + half at position (2 kk + half) ^ (col & 15).
  // V^T operand (transposed read h of k-step kk, d block db): lane p of 16-lane group
  // gq addresses key 16 kk + 4 (gq / 2) + 8 h + p / 4, d = 32 db + 16 (gq % 2) + 4 (p % 4).
  const int gq = lane >> 4;
  const int p16 = lane & 15;
  const int v_key = 4 * (gq >> 1) + (p16 >> 2);
  const int v_chunk_lo = 2 * (gq & 1) + ((p16 >> 1) & 1);  // chunk within the 64-byte block
  int v_off[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
    v_off[db] = kTileBytes + v_key * 256 + ((4 * db + v_chunk_lo) ^ (4 * (p16 >> 2))) * 16 +
                8 * (p16 & 1);

  floatx16 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.f;
  // m: this lane's reference max of the raw scores q.k; every S^T accumulator starts at -m,
  // so the scores leave the matrix cores as s - m and p = 2^(c (s - m)), c = scale * log2 e.
  const float c = a.scale_log2;
  const float lazy_limit = 8.f / c;  // 2^8 in p
  float m = 0.f, l = 0.f;
  floatx16 negm;
#pragma unroll
  for (int r = 0; r < 16; ++r) negm[r] = 0.f;
  const int my_q = wq0 + col;
  const int my_horizon = rq.prefix + my_q;

  // One 64-key tile per step: S^T = K Q^T - m (two 32-key blocks), mask and row max,
  // lazy rescale, P^T = 2^(S^T), O^T += V^T P^T.
  auto compute = [&](int t, int stage, bool first) {
    const int k0 = t * kTileK;
    if (!(wave_active && k0 <= wave_last_key)) return;
    const uint8_t* sb = lds + stage * kStageBytes;
    uint4 kf[2][8];
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
      for (int kk = 0; kk < 8; ++kk)
        kf[T][kk] = *reinterpret_cast<const uint4*>(
            sb + (32 * T + col) * 256 + (((2 * kk + half) ^ (col & 15)) * 16));
    floatx16 s[2];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
#pragma unroll
      for (int T = 0; T < 2; ++T) s[T] = Mfma<DT>::run(kf[T][kk], qreg[kk], kk == 0 ? negm : s[T]);
    uint4 vf[4][4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        lds_u8* vp = (lds_u8*)sb + v_off[db] + 16 * kk * 256;
        const uint2 l2 =
            __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)vp));
        const uint2 h2 = __builtin_bit_cast(
            uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(vp + 8 * 256)));
        vf[kk][db] = make_uint4(l2.x, l2.y, h2.x, h2.y);
      }
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
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx),
                                                        false, false);
      mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));  // max of s - m
    }
    // Lazy rescale: m moves on the first tile (to the row max) and afterwards only when
    // some row's max exceeds it by more than 8 / c, so p = 2^(c (s - m)) <= 2^8 and O / l
    // are rescaled rarely. The first tile of a whole item holds key 0, which each query sees,
    // so mx is finite there; the first tile of a later chunk can lie wholly past a query's
    // horizon (mx = -inf), and that row then keeps m = 0 until a key reaches it.
    if (first || __any(mx > lazy_limit)) {
      const float shift = first ? (mx == -INFINITY ? 0.f : mx) : fmaxf(mx, 0.f);
      // Nothing is accumulated before the first tile; its shift can be any size (every
      // score far below zero makes 2^-shift overflow, and 0 * inf would be NaN).
      const float alpha = first ? 1.f : __builtin_amdgcn_exp2f(-shift * c);
      m += shift;
      l *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[0][r] -= shift;
        s[1][r] -= shift;
        negm[r] = -m;
      }
    }
    uint4 pb[4];
    float ls[4] = {0.f, 0.f, 0.f, 0.f};  // independent partial row sums (fp32 p)
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        float p[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          p[i] = __builtin_amdgcn_exp2f(s[T][8 * hh + i] * c);
          ls[i & 3] += p[i];
        }
        pb[2 * T + hh] = make_uint4(pack2<DT>(p[0], p[1]), pack2<DT>(p[2], p[3]),
                                    pack2<DT>(p[4], p[5]), pack2<DT>(p[6], p[7]));
      }
    l += (ls[0] + ls[1]) + (ls[2] + ls[3]);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] = Mfma<DT>::run(vf[kk][db], pb[kk], o[db]);
  };

  if constexpr (PAGED) {
    if (fast_pages) load_ids(t_begin);
  }
#pragma unroll
  for (int st = 0; st < kAhead; ++st)
    if (st < nt) issue(t_begin + st, st);
  for (int u = 0; u < nt; ++u) {
    wait_tiles_ahead<kCopiesPerTile, kAhead - 1>(min(kAhead - 1, nt - 1 - u));
    __syncthreads();
    if (u + kAhead < nt) issue(t_begin + u + kAhead, (u + kAhead) % STAGES);
    compute(t_begin + u, u % STAGES, u == 0);
  }

  if (!wave_active) return;
  const float row_sum = l + __shfl_xor(l, 32);
  if (pslot >= 0) {
    // Chunk of a split item: O / l and m + log2 l (or 0 and -inf when no key of the
    // chunk reaches this query) for the merge launch. The record keeps the lanes' own
    // order (float4 f = (4 db + g4) * 64 + lane), so each store covers 1 KB contiguously.
    if (my_q >= rq.q_len) return;
    const float inv = row_sum > 0.f ? 1.f / row_sum : 0.f;
    const int64_t rec = static_cast<int64_t>(pslot) * NW + slot_id;
    float* po = a.part_o + rec * (kQPerWave * kD);
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4)
        *reinterpret_cast<float4*>(po + ((4 * db + g4) * 64 + lane) * 4) =
            make_float4(o[db][4 * g4] * inv, o[db][4 * g4 + 1] * inv, o[db][4 * g4 + 2] * inv,
                        o[db][4 * g4 + 3] * inv);
    if (half == 0)
      a.part_lse[rec * kQPerWave + col] =
          row_sum > 0.f ? m * c + __builtin_amdgcn_logf(row_sum) : -INFINITY;
    return;
  }
  // The wave's 32 x 128 output tile goes out as whole 256-byte rows: written to an LDS
  // region no wave reads any more (a stage other than the last tile's: every wave has
  // passed the barrier after finishing the tiles before it; waves 0-3 and 4-7 take two
  // different stages, 8 KB each, 16-byte chunks XOR-swizzled by row so the row
  // reads are conflict-free and the column writes nearly so: rows r and r + 16 share
  // banks), then read back row-major.
  // (Lane-order stores of 16 bytes per query row cost ~4.8 us per item at config 3.)
  const float inv = 1.f / row_sum;
  uint8_t* tile = lds + ((nt + (wave >> 2)) % STAGES) * kStageBytes + (wave & 3) * 8192;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int chunk = (4 * db + g4) ^ (col & 15);
      *reinterpret_cast<uint2*>(tile + col * 256 + chunk * 16 + half * 8) =
          make_uint2(pack2<DT>(o[db][4 * g4] * inv, o[db][4 * g4 + 1] * inv),
                     pack2<DT>(o[db][4 * g4 + 2] * inv, o[db][4 * g4 + 3] * inv));
    }
  const int c16 = lane & 15;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int row = 4 * j + (lane >> 4);
    const uint4 val = *reinterpret_cast<const uint4*>(tile + row * 256 + ((c16 ^ (row & 15)) * 16));
    if (wq0 + row < rq.q_len)
      *reinterpret_cast<uint4*>(a.out + static_cast<int64_t>(rq.q_start + wq0 + row) * a.o_sn +
                                qh * a.o_sh + c16 * 8) = val;
  }
}

// Merge of split items: one workgroup per (split item, wave slot, 32-dim block), eight
// threads per query row of the slot, four dims (one float4 of a record) per thread, so a
// launch spreads over 32 x as many workgroups as split items. Chunks combine by their
// log2-sum-exp, eight at a time so their loads are in flight together (a chunk with
// lse = -inf adds nothing; every query sees key 0, so at least one chunk is finite).
// groups: per split item {request, q_begin, kv_head, head_group}, {first record, count}.
template <int DT, int NW>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillArgs a, const int4* groups,
                                                            int waves_per_head, int hpb) {
  const int gi = blockIdx.x;
  const int slot = blockIdx.y;
  const int db = blockIdx.z;
  const int4 w = groups[2 * gi];
  const int4 cnt = groups[2 * gi + 1];
  const ReqInfo rq = a.reqs[w.x];
  const int group = a.num_q_heads / a.num_kv_heads;
  const int qh = w.z * group + w.w * hpb + slot / waves_per_head;
  const int q = threadIdx.x >> 3;
  const int g4 = (threadIdx.x >> 1) & 3;
  const int h = threadIdx.x & 1;
  const int my_q = w.y + (slot % waves_per_head) * kQPerWave + q;
  if (my_q >= rq.q_len) return;
  // Dims 32 db + 8 g4 + 4 h + i of query q sit in float4 (4 db + g4) * 64 + q + 32 h of a
  // record (the main kernel's lane order).
  const int f = (4 * db + g4) * 64 + q + 32 * h;
  constexpr int kU = 8;
  float mx = -INFINITY, den = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int c0 = 0; c0 < cnt.y; c0 += kU) {
    float lse[kU];
    float4 v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int c = min(c0 + u, cnt.y - 1);
      const int64_t rec = static_cast<int64_t>(cnt.x + c) * NW + slot;
      lse[u] = c0 + u < cnt.y ? a.part_lse[rec * kQPerWave + q] : -INFINITY;
      v[u] = *reinterpret_cast<const float4*>(a.part_o + rec * (kQPerWave * kD) + f * 4);
    }
    float m_new = mx;
#pragma unroll
    for (int u = 0; u < kU; ++u) m_new = fmaxf(m_new, lse[u]);
    if (m_new == -INFINITY) continue;  // no key of these chunks reaches this query yet
    const float corr = __builtin_amdgcn_exp2f(mx - m_new);
    den *= corr;
    acc = make_float4(acc.x * corr, acc.y * corr, acc.z * corr, acc.w * corr);
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const float wgt = __builtin_amdgcn_exp2f(lse[u] - m_new);  // 0 for lse = -inf
      den += wgt;
      acc = make_float4(fmaf(wgt, v[u].x, acc.x), fmaf(wgt, v[u].y, acc.y),
                        fmaf(wgt, v[u].z, acc.z), fmaf(wgt, v[u].w, acc.w));
    }
    mx = m_new;
  }
  const float inv = 1.f / den;
  *reinterpret_cast<uint2*>(a.out + static_cast<int64_t>(rq.q_start + my_q) * a.o_sn +
                            qh * a.o_sh + 32 * db + 8 * g4 + 4 * h) =
      make_uint2(pack2<DT>(acc.x * inv, acc.y * inv), pack2<DT>(acc.z * inv, acc.w * inv));
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

// Waves per prefill workgroup. A batch with a cached prefix (paged) streams long key
// ranges per item, and 8-wave workgroups (one per CU, 256 query rows per item) read each
// K/V tile for twice the rows; a batch without one (ragged, every item a causal triangle
// or part of one) runs 4-wave workgroups, two per CU, so one workgroup's prologue, epilogue
// and barriers overlap the other's tiles (measured: config 3 1.5% faster, the 8 x 1024-token
// Qwen3-8B prompt batch 6% faster; on config 4's long prefixes 8 waves are 5% faster).
// MI355X_PREFILL_WAVES=8 keeps 8 waves for every batch (tuning knob, read once).
int prefill_waves(bool paged) {
  static const bool force8 = [] {
    const char* env = std::getenv("MI355X_PREFILL_WAVES");
    return env && std::atoi(env) == 8;
  }();
  return paged || force8 ? kWaves : 4;
}

bool has_prefix(const int32_t* prefix_host, int64_t batch) {
  for (int64_t i = 0; i < batch; ++i)
    if (prefix_host[i] > 0) return true;
  return false;
}

// q heads per workgroup: all g heads of a kv head when g <= the waves, so each K/V tile
// is fetched once for the whole group.
int heads_per_block(int64_t group, int waves) {
  // MI355X_PREFILL_HPB (1, 2, 4 or 8, at most the group and the waves) overrides the
  // default (tuning knob, read once).
  static const int forced = [] {
    const char* env = std::getenv("MI355X_PREFILL_HPB");
    const int v = env ? std::atoi(env) : 0;
    return (v == 1 || v == 2 || v == 4 || v == 8) ? v : 0;
  }();
  if (forced && forced <= group && forced <= waves && group % forced == 0) return forced;
  return static_cast<int>(std::min<int64_t>(group, waves));
}

}  // namespace

struct PrefillPlan {
  int device = -1;
  int64_t num_q_heads = 0, num_kv_heads = 0, page_size = 0, dtype = 0;
  int64_t batch = 0, total_q = 0, num_items = 0, total_pages = 0;
  bool paged = false;
  int64_t cus = 0;          // compute units of the plan's device
  int64_t num_groups = 0;   // items split along the keys (merged by a second launch)
  int64_t num_records = 0;  // partial records (chunks of split items)
  // Device int32 workspace: [req info 4*B][work 4*items][ranges 4*items][kv_indptr B+1]
  // [last_len B][groups 8*num_groups]
  int64_t o_work = 0, o_ranges = 0, o_indptr = 0, o_last = 0, o_groups = 0;
  Buffer ints, indices, staging, part_o, part_lse;
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
  const int waves = prefill_waves(has_prefix(prefix_host, batch));
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
  // Longest first: the heavy causal tail starts early and the short items fill the gaps.
  // (Grouping the items of one request and kv head on one XCD, for L2 reuse, measured
  // slower on MI355X: the load balance loss outweighed the saved K/V reads.)
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

namespace mi355x {
namespace {
constexpr int64_t kMinChunkTiles = 8;  // keys of a split chunk: at least 8 tiles (512)

// Splits the items of a work list along their keys when the batch is too small to fill the
// chip (the reference's prefill plan splits KV the same way for low parallelism,
// flashinfer_plan_run.cu:243-274,312-316): when the longest item holds more than twice the
// mean per-CU share of tiles, every item longer than max(8, that share) becomes
// ceil(tiles / chunk) chunks of near-equal length. Unsplit items keep range {0, tiles, -1};
// chunk j of split item g gets {first, end, record} with records consecutive per item.
// Output order: longest chunk or item first.
struct SplitPlan {
  std::vector<int32_t> work, ranges, groups;  // 4, 4 and 8 ints per entry
  int64_t records = 0;
};
SplitPlan split_items(const std::vector<int32_t>& base, const int32_t* q_host,
                      const int32_t* prefix_host, int64_t num_q_heads, int64_t num_kv_heads,
                      int64_t cus, int waves) {
  const int64_t n = static_cast<int64_t>(base.size() / 4);
  const int hpb = heads_per_block(num_q_heads / num_kv_heads, waves);
  const int64_t bq = kQPerWave * (waves / hpb);
  std::vector<int64_t> tiles(n);
  int64_t total = 0, longest = 0;
  for (int64_t i = 0; i < n; ++i) {
    const int r = base[4 * i];
    const int64_t q_len = q_host[r + 1] - q_host[r];
    const int64_t horizon = prefix_host[r] + std::min<int64_t>(base[4 * i + 1] + bq, q_len);
    tiles[i] = (horizon + kTileK - 1) / kTileK;
    total += tiles[i];
    longest = std::max(longest, tiles[i]);
  }
  const int64_t share = (total + cus - 1) / std::max<int64_t>(cus, 1);
  // MI355X_PREFILL_SPLIT=0 turns splitting off (tuning knob, read once).
  static const bool enabled = [] {
    const char* env = std::getenv("MI355X_PREFILL_SPLIT");
    return !(env && std::strcmp(env, "0") == 0);
  }();
  const bool split = enabled && longest > 2 * share && longest > 2 * kMinChunkTiles;
  const int64_t chunk = std::max(kMinChunkTiles, share);
  struct Entry {
    int64_t cost;
    int64_t item, first, end, record;
  };
  std::vector<Entry> entries;
  SplitPlan out;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t k = split && tiles[i] > chunk ? (tiles[i] + chunk - 1) / chunk : 1;
    if (k == 1) {
      entries.push_back({tiles[i], i, 0, tiles[i], -1});
      continue;
    }
    out.groups.insert(out.groups.end(), base.begin() + 4 * i, base.begin() + 4 * i + 4);
    out.groups.insert(out.groups.end(), {static_cast<int32_t>(out.records),
                                         static_cast<int32_t>(k), 0, 0});
    for (int64_t j = 0; j < k; ++j) {
      const int64_t first = tiles[i] * j / k, end = tiles[i] * (j + 1) / k;
      entries.push_back({end - first, i, first, end, out.records++});
    }
  }
  std::stable_sort(entries.begin(), entries.end(),
                   [](const Entry& x, const Entry& y) { return x.cost > y.cost; });
  for (const Entry& e : entries) {
    out.work.insert(out.work.end(), base.begin() + 4 * e.item, base.begin() + 4 * e.item + 4);
    out.ranges.insert(out.ranges.end(), {static_cast<int32_t>(e.first),
                                         static_cast<int32_t>(e.end),
                                         static_cast<int32_t>(e.record), 0});
  }
  return out;
}
}  // namespace
}  // namespace mi355x

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
      if (int64_t(prefix_host[i]) + q_host[i + 1] - q_host[i] >= kMaxKvLen) {
        set_error("prefill sequence longer than 4194303 tokens");
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
    const int64_t n_base =
        mi355x_prefill_schedule(q_host, prefix_host, batch, num_q_heads, num_kv_heads, nullptr, 0);
    if (n_base <= 0 || n_base > std::numeric_limits<int32_t>::max() / 64) {
      set_error("prefill work list is empty or too large");
      return nullptr;
    }
    if (!plan->cus) {
      int cus = 0;
      st = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
      if (st != hipSuccess || cus <= 0) {
        hip_error(st, "hipDeviceGetAttribute");
        return nullptr;
      }
      plan->cus = cus;
    }
    std::vector<int32_t> base(4 * n_base);
    mi355x_prefill_schedule(q_host, prefix_host, batch, num_q_heads, num_kv_heads, base.data(),
                            n_base);
    const SplitPlan sp =
        split_items(base, q_host, prefix_host, num_q_heads, num_kv_heads, plan->cus,
                    prefill_waves(paged));
    const int64_t n_items = static_cast<int64_t>(sp.work.size() / 4);
    const int64_t n_groups = static_cast<int64_t>(sp.groups.size() / 8);
    if (n_items > std::numeric_limits<int32_t>::max() / 64) {
      set_error("prefill work list is empty or too large");
      return nullptr;
    }
    const int64_t o_work = 4 * batch;
    const int64_t o_ranges = o_work + 4 * n_items;
    const int64_t o_indptr = o_ranges + 4 * n_items;
    const int64_t o_last = o_indptr + batch + 1;
    const int64_t o_groups = (o_last + batch + 3) / 4 * 4;  // int4-aligned
    const int64_t total_ints = o_groups + 8 * n_groups;
    st = hipEventSynchronize(plan->upload_done);
    if (st != hipSuccess) {
      hip_error(st, "prefill upload fence");
      return nullptr;
    }
    const size_t rec_bytes =
        static_cast<size_t>(sp.records) * prefill_waves(paged) * kQPerWave * 4;
    if ((st = plan->ints.reserve(total_ints * 4, plan->allocations)) != hipSuccess ||
        (st = plan->staging.reserve(total_ints * 4, plan->allocations)) != hipSuccess ||
        (sp.records && (st = plan->part_o.reserve(rec_bytes * kD, plan->allocations)) !=
                           hipSuccess) ||
        (sp.records && (st = plan->part_lse.reserve(rec_bytes, plan->allocations)) !=
                           hipSuccess)) {
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
    std::memcpy(host + o_work, sp.work.data(), sp.work.size() * 4);
    std::memcpy(host + o_ranges, sp.ranges.data(), sp.ranges.size() * 4);
    if (n_groups) std::memcpy(host + o_groups, sp.groups.data(), sp.groups.size() * 4);
    st = hipMemcpyAsync(plan->ints.ptr, host, total_ints * 4, hipMemcpyHostToDevice, s);
    if (st != hipSuccess) {
      hip_error(st, "prefill metadata upload");
      return nullptr;
    }
    if (paged) {
      if ((st = plan->indices.reserve((total_pages + 4) * 4, plan->allocations)) !=
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
    plan->num_groups = n_groups;
    plan->num_records = sp.records;
    plan->total_pages = total_pages;
    plan->paged = paged;
    plan->o_work = o_work;
    plan->o_ranges = o_ranges;
    plan->o_indptr = o_indptr;
    plan->o_last = o_last;
    plan->o_groups = o_groups;
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

// Plan facts: out6 = {batch, total_q, paged, num_items, total_pages, items split along keys}.
extern "C" const char* mi355x_prefill_plan_info(const void* plan, int64_t* out6) {
  if (!plan || !out6) return set_error("mi355x_prefill_plan_info: null argument");
  const auto* p = static_cast<const PrefillPlan*>(plan);
  out6[0] = p->batch;
  out6[1] = p->total_q;
  out6[2] = p->paged ? 1 : 0;
  out6[3] = p->num_items;
  out6[4] = p->total_pages;
  out6[5] = p->num_groups;
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
template <int DT, int HPB, int NW, bool PAGED>
void launch_prefill(const PrefillArgs& a, hipStream_t s) {
  prefill_kernel<DT, HPB, PAGED, NW>
      <<<dim3(static_cast<uint32_t>(a.num_items)), dim3(64 * NW), 0, s>>>(a);
}
template <int DT, bool PAGED>
void launch_waves8(const PrefillArgs& a, int hpb, hipStream_t s) {
  if (hpb == 1) launch_prefill<DT, 1, kWaves, PAGED>(a, s);
  else if (hpb == 2) launch_prefill<DT, 2, kWaves, PAGED>(a, s);
  else if (hpb == 4) launch_prefill<DT, 4, kWaves, PAGED>(a, s);
  else launch_prefill<DT, 8, kWaves, PAGED>(a, s);
}
template <int DT>
void launch_dt(const PrefillArgs& a, int hpb, int waves, bool paged, const int4* groups,
               int64_t num_groups, hipStream_t s) {
  if (waves == 4) {  // ragged batches only
    if (hpb == 1) launch_prefill<DT, 1, 4, false>(a, s);
    else if (hpb == 2) launch_prefill<DT, 2, 4, false>(a, s);
    else launch_prefill<DT, 4, 4, false>(a, s);
    if (num_groups)
      prefill_merge_kernel<DT, 4><<<dim3(static_cast<uint32_t>(num_groups), 4, kD / 32),
                                    dim3(256), 0, s>>>(a, groups, 4 / hpb, hpb);
    return;
  }
  if (paged) launch_waves8<DT, true>(a, hpb, s);
  else launch_waves8<DT, false>(a, hpb, s);
  if (num_groups)
    prefill_merge_kernel<DT, kWaves><<<dim3(static_cast<uint32_t>(num_groups), kWaves, kD / 32),
                                       dim3(256), 0, s>>>(a, groups, kWaves / hpb, hpb);
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
  a.ranges = reinterpret_cast<const int4*>(ints + p.o_ranges);
  a.part_o = static_cast<float*>(p.part_o.ptr);
  a.part_lse = static_cast<float*>(p.part_lse.ptr);
  a.indices = static_cast<const int32_t*>(p.indices.ptr);
  a.num_items = static_cast<int32_t>(p.num_items);
  a.num_q_heads = static_cast<int32_t>(num_q_heads);
  a.num_kv_heads = static_cast<int32_t>(num_kv_heads);
  a.page_size = static_cast<int32_t>(p.paged ? page_size : 1);
  a.scale_log2 = (1.0f / std::sqrt(static_cast<float>(kD))) * kLog2e;
  const int waves = prefill_waves(p.paged);
  const int hpb = heads_per_block(num_q_heads / num_kv_heads, waves);
  auto s = static_cast<hipStream_t>(stream);
  const int4* groups = reinterpret_cast<const int4*>(ints + p.o_groups);
  if (dtype == 0)
    launch_dt<0>(a, hpb, waves, p.paged, groups, p.num_groups, s);
  else
    launch_dt<1>(a, hpb, waves, p.paged, groups, p.num_groups, s);
  return launch_status("prefill_kernel");
}
