// Paged decode attention for gfx950: per-forward plan (page metadata + split-KV
// work list), the decode kernel and the split-KV merge kernel.
//
// Reference path this replaces:
//   plan:  sglang_flashinfer_prepare   src/models/attention/flashinfer_bridge.cpp:61-185
//          pack_decode_metadata        src/models/attention/flashinfer_plan_run.cu:24-34
//          DecodePlan (work estimation) flashinfer_plan_run.cu:74-125
//   run:   sglang_flashinfer_decode    flashinfer_bridge.cpp:201-240
//          BatchDecodeWithPagedKVCacheDispatched  flashinfer_plan_run.cu:127-173
//   math:  o[b,h] = softmax_j(q[b,h] . k[j,h/g] * sm_scale) v[j,h/g], j over the
//          request's cache_seqlens[b] tokens, sm_scale = 1/sqrt(128)
//          (backend.rs:1375-1420 decode_with_cache_padded is the libtorch restatement).
//
// Page metadata is the reference's closed form, bit for bit:
//   indptr[0] = 0, indptr[r+1] = indptr[r] + ceil(len[r] / P)
//   indices[indptr[r] + c] = block_table[r * stride + c], c < ceil(len[r] / P)
//   last_page_len[r] = (len[r] - 1) % P + 1
//
// Split-KV schedule (our own design for 256 CUs): the grid's workgroups each take
// an equal share of the batch's work, counted in the kernel's 16-token tiles plus a
// fixed cost per work item ("stream-K" over the flattened tile list), or whole
// requests when that is cheaper than the split and its merge launch; the requests a
// share touches become its work items. A request held by one item writes its output
// directly; a request cut into several items writes normalised fp32 partials +
// log2-sum-exp that a small merge kernel combines.
// (Merging inside the last-arriving workgroup needs an agent-scope release per
// workgroup, i.e. an L2 write-back on every XCD, and measured ~5x slower than the
// extra launch.)
//
// Kernels. decode_dma_kernel (kv-head slices of 4 or 8 heads, the common case):
// one 8-wave workgroup per CU streams 16-token tiles of whole K and V rows into a
// 2-deep LDS ring with direct global -> LDS copies; wave w computes kv head w.
// decode_kernel (other head counts): one wave per kv head loads its 256-byte row
// slices straight into registers.
#include <algorithm>
#include <functional>
#include <type_traits>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <memory>
#include <vector>

#include "common.h"

namespace mi355x {
namespace {

constexpr int kHeadDim = 128;
constexpr int kTokensPerLaneGroup = 4;  // tokens per 16-lane group per loop trip
constexpr int kTileTokens = 32;  // chunk granularity: a multiple of every tile size (4 * U)
constexpr int kMaxWavesPerBlock = 8;
// decode_dma_kernel shape (measured on MI355X at configs 2 and 5: 16-token tiles in a
// 2-deep ring, one 8-wave workgroup per CU, beat 8-token tiles with 3-4 stages and
// 4-wave workgroups two per CU).
constexpr int kDmaTile = 16;           // tokens per LDS tile
constexpr int kDmaStages = 2;          // LDS ring depth
constexpr int kDmaMaxEntries = 2048;   // page entries of one work item held in LDS
static_assert(kDmaMaxEntries % 64 == 0, "entries are staged 64 at a time");
constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// Device buffer with geometric growth, matching the reference workspace rule
// (flashinfer_plan_run.cu:47-65): grow x2 from 64 KiB, count allocations.
// ---------------------------------------------------------------------------
struct DeviceBuffer {
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
    if (!pinned) {
      st = hipMemset(fresh, 0, grown);
      if (st != hipSuccess) {
        (void)hipFree(fresh);
        return st;
      }
    }
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
  ~DeviceBuffer() { release(); }
};

// int32 workspace layout (device and pinned staging share it):
//   [0]                  number of workgroups (per kv-head slice)
//   [1]                  number of work items
//   [4, 4+B+1)           indptr
//   [o_work, +4*cap)     work items {request, token_begin, token_end, partial}
//   [o_merge, +2*B)      per-request {first partial, chunk count}
//   [o_wg, +wgs+1)       first work item of each workgroup
//   [o_wgrec, +32*cap)   per-workgroup start record (kWgRec ints, 128-byte aligned):
//                        {first item, item end, request, token_begin, token_end,
//                         partial, page base, 0} of its first item, then the KV slots
//                        of that item's first kDmaTile tokens (clamped to the item)
constexpr int kWgRec = 32;
constexpr int kWgRecSlots = 8;  // offset of the slots within a record
static_assert(kWgRecSlots + kDmaTile <= kWgRec, "a start record holds one tile's slots");
struct IntLayout {
  int64_t o_indptr, o_work, o_merge, o_wg, o_wgrec, total;
  static IntLayout make(int64_t rows, int64_t items_cap, int64_t wg_cap) {
    IntLayout l{};
    l.o_indptr = 4;
    l.o_work = (l.o_indptr + rows + 1 + 3) / 4 * 4;
    l.o_merge = l.o_work + 4 * items_cap;
    l.o_wg = l.o_merge + 2 * rows;
    l.o_wgrec = (l.o_wg + wg_cap + 1 + kWgRec - 1) / kWgRec * kWgRec;
    l.total = l.o_wgrec + kWgRec * wg_cap;
    return l;
  }
};

}  // namespace

struct DecodePlan {
  int device = -1;
  int64_t num_q_heads = 0, num_kv_heads = 0, head_dim = 0, page_size = 0, dtype = 0;
  bool graph = false;
  int64_t graph_rows = 0, graph_columns = 0;
  // Current plan facts.
  int64_t batch = 0, total_pages = 0, num_items = 0, chunk_tokens = 0, items_capacity = 0;
  int64_t num_wgs = 0, wg_capacity = 0;
  int64_t cus = 0;
  IntLayout layout{};
  DeviceBuffer ints, indices, last_len, partial_o, partial_lse;
  DeviceBuffer staging;
  hipEvent_t upload_done = nullptr;
  uint64_t allocations = 0;
  std::vector<int32_t> host_lengths;

  DecodePlan() { staging.pinned = true; }
  ~DecodePlan() {
    if (upload_done) {
      (void)hipEventSynchronize(upload_done);
      (void)hipEventDestroy(upload_done);
    }
  }
};

namespace {

// ---------------------------------------------------------------------------
// Host planner: split-KV work list. Pure host code.
// ---------------------------------------------------------------------------
// Resident waves per CU the split-KV schedule aims to fill. Override with
// MI355X_DECODE_WAVES_PER_CU (tuning knob; read once).
int64_t waves_per_cu_target() {
  static const int64_t value = [] {
    const char* env = std::getenv("MI355X_DECODE_WAVES_PER_CU");
    const long v = env ? std::strtol(env, nullptr, 10) : 0;
    return v > 0 ? static_cast<int64_t>(v) : int64_t(32);
  }();
  return value;
}

// Waves (= kv heads) per decode workgroup. Override with
// MI355X_DECODE_WAVES_PER_BLOCK (1..8; tuning knob, read once).
int64_t waves_per_block(int64_t num_kv_heads) {
  static const int64_t cap = [] {
    const char* env = std::getenv("MI355X_DECODE_WAVES_PER_BLOCK");
    const long v = env ? std::strtol(env, nullptr, 10) : 0;
    return (v >= 1 && v <= kMaxWavesPerBlock) ? static_cast<int64_t>(v)
                                              : static_cast<int64_t>(kMaxWavesPerBlock);
  }();
  return std::min<int64_t>(num_kv_heads, cap);
}

int64_t target_items_for(int64_t cus, int64_t num_kv_heads) {
  const int64_t waves = waves_per_block(num_kv_heads);
  const int64_t grid_y = (num_kv_heads + waves - 1) / waves;
  const int64_t per_cu = std::max<int64_t>(1, waves_per_cu_target() / waves);
  return std::max<int64_t>(1, cus * per_cu / grid_y);
}

// decode_dma_kernel for kv-head slices of 4 or 8 heads (tuning knobs, read once:
// MI355X_DECODE_DMA=0 selects decode_kernel everywhere, MI355X_DECODE_DMA_W=4|8
// forces the slice width).
bool dma_enabled() {
  static const bool on = [] {
    const char* env = std::getenv("MI355X_DECODE_DMA");
    return !(env && std::strcmp(env, "0") == 0);
  }();
  return on;
}

int64_t dma_lds_bytes(int64_t waves) {
  return int64_t(kDmaStages) * 2 * kDmaTile * waves * 256 + int64_t(kDmaMaxEntries) * 4;
}

// How a decode launch is laid out for a kv-head count and page size.
struct LaunchShape {
  bool dma;            // decode_dma_kernel, else decode_kernel
  int64_t waves;       // waves (kv heads) per workgroup
  int64_t grid_y;      // kv-head slices
  int64_t workgroups;  // split-KV workgroups per slice: the schedule's target
  int64_t max_item;    // most tokens of one work item
  int64_t tile;        // tokens per kernel tile: the schedule's unit of work
  int64_t wg_capacity;
};

LaunchShape launch_shape(int64_t cus, int64_t num_kv_heads, int64_t page_size) {
  LaunchShape s{};
  static const int64_t forced_w = [] {
    const char* env = std::getenv("MI355X_DECODE_DMA_W");
    const int v = env ? std::atoi(env) : 0;
    return int64_t(v == 4 || v == 8 ? v : 0);
  }();
  const int64_t w =
      forced_w && num_kv_heads % forced_w == 0 ? forced_w : std::min<int64_t>(num_kv_heads, kMaxWavesPerBlock);
  s.dma = dma_enabled() && (w == 4 || w == 8) && num_kv_heads % w == 0;
  if (s.dma) {
    s.waves = w;
    s.grid_y = num_kv_heads / w;
    const int64_t per_cu = std::max<int64_t>(1, (160 * 1024) / dma_lds_bytes(w));
    s.workgroups = std::max<int64_t>(1, cus * per_cu / s.grid_y);
    s.max_item = int64_t(kDmaMaxEntries - 1) * page_size;  // its page entries fit in LDS
    s.tile = kDmaTile;
  } else {
    s.waves = waves_per_block(num_kv_heads);
    s.grid_y = (num_kv_heads + s.waves - 1) / s.waves;
    s.workgroups = target_items_for(cus, num_kv_heads);
    s.max_item = std::numeric_limits<int32_t>::max();
    s.tile = kTileTokens;
  }
  // Every workgroup but the last takes more than share - 32 >= 3/4 share tokens.
  s.wg_capacity = s.workgroups + s.workgroups / 3 + 2;
  return s;
}

// Items: one per request a share touches (<= workgroups + rows) plus the cuts at
// max_item for rows of up to `row_tokens` tokens.
int64_t items_capacity_for(const LaunchShape& s, int64_t rows, int64_t row_tokens) {
  return s.wg_capacity + rows * (1 + (row_tokens + s.max_item - 1) / s.max_item);
}

// Balanced split-KV ("stream-K" over the flattened tile list): the workgroups of the
// grid each take an equal share of the batch's work, walking the requests in order. Work
// is counted in the kernel's tiles (`tile` tokens; a request's last tile may be partial)
// plus a fixed cost per work item, because a workgroup's time is set by the tiles it
// streams and the prologue of each item it starts (its page entries and query rows are
// loaded before its first copies issue), and a workgroup holding more than its share
// delays the whole launch. Cuts fall on tile boundaries, so no share pays for a partial
// tile in the middle of a request. A workgroup's share becomes one work item per request
// it touches; a request cut into several items gets normalised partials that the merge
// kernel combines, one held by a single item writes its output directly. An item holds
// at most `max_item` tokens.
// Fills work (4 ints per item), merge (2 ints per request) and, when wg is not NULL,
// wg[i] = first item of workgroup i (wg[workgroups] = item count). Returns the item
// count, or -1 when a capacity is too small.
int64_t schedule(const int32_t* lengths, int64_t batch, int64_t workgroups, int64_t max_item,
                 int64_t tile, int32_t* work, int64_t capacity, int32_t* merge,
                 int64_t* share_out, int32_t* wg = nullptr, int64_t wg_capacity = 0,
                 int64_t* wgs_out = nullptr) {
  constexpr int64_t kMinShareTokens = 128;
  constexpr int64_t kUnit = 8;  // cost units per tile
  // An item's prologue in cost units: 9/8 of a tile, as measured (per-workgroup end
  // times at configs 2 and 5 fit 2.5-2.6 us per tile + 2.4-2.9 us per item). With it,
  // requests of nearly equal length (the config-5 decode batches) are no longer cut
  // just to even out a tile or two: 236.5 vs 244.4 us per launch there, and config 2
  // within 0.3 us. Override with MI355X_DECODE_ITEM_COST (eighths of a tile; tuning
  // knob, read once).
  static const int64_t kItemCost = [] {
    const char* env = std::getenv("MI355X_DECODE_ITEM_COST");
    const long v = env ? std::strtol(env, nullptr, 10) : -1;
    return v >= 0 ? static_cast<int64_t>(v) : int64_t(9);
  }();
  // The merge launch and the partials' traffic, in cost units (~2 tiles: config 5's
  // decode launch takes 4.3 us longer with six requests split than with none).
  constexpr int64_t kMergeCost = 16;
  const int64_t max_item_tiles = std::max<int64_t>(1, max_item / tile);
  // Tiles per request, computed once (the walks below run a dozen times per plan).
  std::vector<int32_t> tiles_of(batch);
  int64_t total = 0;
  for (int64_t r = 0; r < batch; ++r) {
    tiles_of[r] = static_cast<int32_t>((lengths[r] + tile - 1) / tile);
    total += tiles_of[r];
  }
  const int64_t min_share = std::max<int64_t>(1, kMinShareTokens / tile) * kUnit;
  // Smallest share (cost units) whose walk needs at most `workgroups` workgroups: start
  // from the tile-only bound and add item costs until the walk fits.
  int64_t share = std::max((total * kUnit + workgroups - 1) / workgroups, min_share);
  // One walk at a given share: 0 when it fits, 1 when it needs more than `wg_limit`
  // workgroups, 2 when the item capacity is too small.
  const int64_t wg_limit = wg ? wg_capacity : workgroups + workgroups / 3 + 2;
  int64_t max_load = 0;  // largest workgroup load of the last walk, in cost units
  // `write` (std::true_type / std::false_type): fill the work list and workgroup starts,
  // or only count (the search below).
  auto walk = [&](int64_t share_units, int64_t& items, int64_t& wgs, auto write) -> int {
    constexpr bool kWrite = decltype(write)::value;
    items = 0;
    wgs = 0;
    max_load = 0;
    int64_t r = 0, pos = 0;  // request, tile within it
    while (r < batch) {
      if (wgs >= wg_limit) return 1;
      if (kWrite && wg) wg[wgs] = static_cast<int32_t>(items);
      ++wgs;
      int64_t budget = share_units;
      while (r < batch) {
        const int64_t tiles = tiles_of[r];
        const int64_t take = std::min(std::min(budget / kUnit, tiles - pos), max_item_tiles);
        if (take <= 0 && tiles > 0) break;
        if (items >= capacity) return 2;
        if constexpr (kWrite) {
          work[4 * items + 0] = static_cast<int32_t>(r);
          work[4 * items + 1] = static_cast<int32_t>(pos * tile);
          work[4 * items + 2] =
              static_cast<int32_t>(std::min<int64_t>((pos + take) * tile, lengths[r]));
        }
        ++items;
        budget -= take * kUnit + kItemCost;
        pos += take;
        if (pos == tiles) {
          ++r;
          pos = 0;
        }
      }
      max_load = std::max(max_load, share_units - budget);
    }
    return 0;
  };
  // A share this large puts every request in one workgroup's items, so the search ends.
  const int64_t everything = total * kUnit + (batch + 1) * kItemCost + kUnit;
  // The workgroup count of a walk does not grow with the share: find the smallest share
  // that fits by an exponential then a binary search (about a dozen walks).
  int64_t items = 0, wgs = 0;
  auto fits = [&](int64_t share_units, int& status) {
    status = walk(share_units, items, wgs, std::false_type{});
    return status == 0 && (wgs <= workgroups || share_units >= everything);
  };
  int status = 0;
  if (!fits(share, status)) {
    if (status == 2) return -1;
    // First guess: every request and every workgroup boundary adds one item.
    int64_t lo = share, hi = share;
    int64_t step = std::max<int64_t>(
        kUnit, ((batch + workgroups) * kItemCost + workgroups - 1) / workgroups);
    for (;;) {  // lo does not fit; find a hi that does
      hi = std::min(everything, lo + step);
      if (fits(hi, status)) break;
      if (status == 2 || hi >= everything) return -1;
      lo = hi;
      step *= 2;
    }
    while (hi - lo > 1) {
      const int64_t mid = lo + (hi - lo) / 2;
      if (fits(mid, status)) {
        hi = mid;
      } else {
        if (status == 2) return -1;
        lo = mid;
      }
    }
    share = hi;
  }
  if (walk(share, items, wgs, std::true_type{}) != 0) return -1;
  // The alternative of whole requests, one item each, placed longest first on the least
  // loaded workgroup: no partials and no merge launch, which outweighs a somewhat longer
  // longest workgroup (batches of nearly equal requests, such as config 5's decode
  // steps: 230.7 us per launch whole against 236.5 balanced and 244.4 with the item cost
  // at 6/8 of a tile).
  const bool split = items > batch;
  bool whole = split && wg_limit >= std::min(batch, workgroups);
  for (int64_t r = 0; whole && r < batch; ++r) whole = lengths[r] <= max_item;
  if (whole) {
    const int64_t bins = std::min(batch, workgroups);
    std::vector<int64_t> bin_of(batch);
    int64_t whole_load = 0;
    if (batch <= workgroups) {  // a workgroup per request
      for (int64_t r = 0; r < batch; ++r) {
        bin_of[r] = r;
        whole_load = std::max(whole_load, tiles_of[r] * kUnit + kItemCost);
      }
    } else {
      std::vector<int64_t> order(batch);
      for (int64_t r = 0; r < batch; ++r) order[r] = r;
      std::stable_sort(order.begin(), order.end(),
                       [&](int64_t x, int64_t y) { return tiles_of[x] > tiles_of[y]; });
      // Min-heap of (load, bin).
      std::vector<std::pair<int64_t, int64_t>> heap;
      heap.reserve(bins);
      for (int64_t b = 0; b < bins; ++b) heap.emplace_back(0, b);
      for (const int64_t r : order) {
        std::pop_heap(heap.begin(), heap.end(), std::greater<>());
        auto& top = heap.back();
        top.first += tiles_of[r] * kUnit + kItemCost;
        whole_load = std::max(whole_load, top.first);
        bin_of[r] = top.second;
        std::push_heap(heap.begin(), heap.end(), std::greater<>());
      }
    }
    if (whole_load <= max_load + kMergeCost && batch <= capacity) {
      // Items grouped by bin (requests in their original order within a bin).
      std::vector<int64_t> first(bins + 1, 0);
      for (int64_t r = 0; r < batch; ++r) ++first[bin_of[r] + 1];
      for (int64_t b = 0; b < bins; ++b) first[b + 1] += first[b];
      std::vector<int64_t> next(first.begin(), first.end() - 1);
      for (int64_t r = 0; r < batch; ++r) {
        const int64_t i = next[bin_of[r]]++;
        work[4 * i + 0] = static_cast<int32_t>(r);
        work[4 * i + 1] = 0;
        work[4 * i + 2] = lengths[r];
      }
      if (wg)
        for (int64_t b = 0; b < bins; ++b) wg[b] = static_cast<int32_t>(first[b]);
      items = batch;
      wgs = bins;
      share = whole_load;
    }
  }
  if (wg) wg[wgs] = static_cast<int32_t>(items);
  // Items of a request are consecutive: count them and assign partial slots.
  int64_t partials = 0;
  for (int64_t i = 0; i < items;) {
    const int32_t req = work[4 * i];
    int64_t n = 0;
    while (i + n < items && work[4 * (i + n)] == req) ++n;
    merge[2 * req] = static_cast<int32_t>(n > 1 ? partials : -1);
    merge[2 * req + 1] = static_cast<int32_t>(n);
    for (int64_t c = 0; c < n; ++c)
      work[4 * (i + c) + 3] = static_cast<int32_t>(n > 1 ? partials + c : -1);
    if (n > 1) partials += n;
    i += n;
  }
  *share_out = share / kUnit * tile;
  if (wgs_out) *wgs_out = wgs;
  return items;
}

// ---------------------------------------------------------------------------
// Page metadata pack: one workgroup per request.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_page_metadata(const int32_t* __restrict__ table,
                                                          const int32_t* __restrict__ lengths,
                                                          const int32_t* __restrict__ indptr,
                                                          int32_t* __restrict__ indices,
                                                          int32_t* __restrict__ last_len,
                                                          int64_t stride, int32_t page_size,
                                                          int32_t* __restrict__ recs,
                                                          int32_t wgs, int32_t rows) {
  const int row = blockIdx.x;
  // Workgroup `row`'s start record: the KV slots of its first item's first tile, read
  // from the block table (tokens past the item clamp to its last, as the decode kernels
  // clamp them). The planner wrote the rest of the record.
  if (row < wgs && threadIdx.x < kDmaTile) {
    int32_t* r = recs + kWgRec * row;
    if (r[0] < r[1]) {
      const int req = r[2], beg = r[3], end = r[4];
      const int tok = min(beg + static_cast<int>(threadIdx.x), end - 1);
      const uint32_t page = static_cast<uint32_t>(table[req * stride + tok / page_size]);
      r[kWgRecSlots + threadIdx.x] = static_cast<int32_t>(
          page * static_cast<uint32_t>(page_size) + static_cast<uint32_t>(tok % page_size));
    }
  }
  if (row >= rows) return;
  const int begin = indptr[row];
  const int pages = indptr[row + 1] - begin;
  if (threadIdx.x == 0) last_len[row] = (lengths[row] - 1) % page_size + 1;
  const int32_t* src = table + row * stride;
  for (int c = threadIdx.x; c < pages; c += blockDim.x) indices[begin + c] = src[c];
}


// ---------------------------------------------------------------------------
// Decode kernel.
// ---------------------------------------------------------------------------
struct DecodeArgs {
  const uint16_t* q;
  int64_t q_stride_n, q_stride_h;
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  uint16_t* out;
  int64_t out_stride_n, out_stride_h;
  const int32_t* ints;  // workspace (num_items, indptr, work, merge)
  int32_t o_indptr, o_work, o_merge, o_wg, o_wgrec;
  const int32_t* indices;
  float* partial_o;
  float* partial_lse;
  int32_t num_q_heads, num_kv_heads, page_size;
  float scale_log2;  // sm_scale * log2(e)
};

// 8-element dot product of packed 16-bit vectors with fp32 accumulation
// (v_dot2c_f32_bf16 / v_dot2c_f32_f16).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

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

template <int DT>
__device__ __forceinline__ float dot8(const uint4& a, const uint4& b) {
  float s = dot2<DT>(a.x, b.x, 0.f);
  s = dot2<DT>(a.y, b.y, s);
  s = dot2<DT>(a.z, b.z, s);
  s = dot2<DT>(a.w, b.w, s);
  return s;
}

template <bool P1>
__device__ __forceinline__ int64_t slot_of(const int32_t* pages, int t, int page_size) {
  if constexpr (P1) {
    return pages[t];
  } else {
    return static_cast<int64_t>(pages[t / page_size]) * page_size + t % page_size;
  }
}

// {a.lo16, b.lo16} and {a.hi16, b.hi16} (v_perm_b32).
__device__ __forceinline__ uint32_t pair_lo(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t pair_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// Online-softmax update of one lane group with U tokens of K/V (U even).
// QK: v_dot2 on packed q/k words + a 16-lane DPP sum. PV: the V words of two
// tokens are re-paired per dim (v_perm) and accumulated with one v_dot2 per
// dim against the packed pair of their probabilities, so V is never unpacked.
template <int DT, int G, int U>
__device__ __forceinline__ void consume(const uint4 (&qv)[G], const uint4 (&kr)[U],
                                       const uint4 (&vr)[U], const bool (&valid)[U],
                                       float scale_log2, float (&m)[G], float (&l)[G],
                                       float (&o)[G][8]) {
  static_assert(U % 2 == 0, "tokens are consumed in pairs");
  // Per dim pair (2k, 2k+1) and token pair: words {a[2k], b[2k]}, {a[2k+1], b[2k+1]}.
  uint32_t vp[U / 2][8];
#pragma unroll
  for (int u = 0; u < U; u += 2) {
    const uint32_t a[4] = {vr[u].x, vr[u].y, vr[u].z, vr[u].w};
    const uint32_t b[4] = {vr[u + 1].x, vr[u + 1].y, vr[u + 1].z, vr[u + 1].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      vp[u / 2][2 * k] = pair_lo(a[k], b[k]);
      vp[u / 2][2 * k + 1] = pair_hi(a[k], b[k]);
    }
  }
  float sc[G * U];
#pragma unroll
  for (int gi = 0; gi < G; ++gi)
#pragma unroll
    for (int u = 0; u < U; ++u) sc[gi * U + u] = dot8<DT>(qv[gi], kr[u]);
  row16_sum_n<G * U>(sc);
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    float s[U];
    float mx = m[gi];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      s[u] = valid[u] ? sc[gi * U + u] * scale_log2 : -INFINITY;
      mx = fmaxf(mx, s[u]);
    }
    const float corr = __builtin_amdgcn_exp2f(m[gi] - mx);
    m[gi] = mx;
    float psum = 0.f;
    uint32_t pp[U / 2];
#pragma unroll
    for (int u = 0; u < U; u += 2) {
      const float p0 = __builtin_amdgcn_exp2f(s[u] - mx);
      const float p1 = __builtin_amdgcn_exp2f(s[u + 1] - mx);
      psum += p0 + p1;
      pp[u / 2] = Elem<DT>::pack2(p0, p1);
    }
    l[gi] = l[gi] * corr + psum;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float acc = o[gi][i] * corr;
#pragma unroll
      for (int u = 0; u < U / 2; ++u) acc = dot2<DT>(vp[u][i], pp[u], acc);
      o[gi][i] = acc;
    }
  }
}

// Element offset of token t's row: slot * row_elems as one 32x32->64 multiply
// (slots < 2^31, rows < 2^32 elements).
template <bool P1>
__device__ __forceinline__ uint64_t slot_offset(const int32_t* pages, int t, int page_size,
                                                uint32_t row_elems) {
  uint32_t slot;
  if constexpr (P1) {
    slot = static_cast<uint32_t>(pages[t]);
  } else {
    slot = static_cast<uint32_t>(pages[t / page_size]) * static_cast<uint32_t>(page_size) +
           static_cast<uint32_t>(t % page_size);
  }
  return static_cast<uint64_t>(slot) * row_elems;
}

// One workgroup = one (request, token chunk) work item; wave w handles kv head
// blockIdx.y * waves + w and its G query heads. Inside a wave, lane group
// grp = lane / 16 takes tokens t0 + 4 u + grp (u < U) and each lane owns 8 of
// the 128 dims. Slot offsets of the next tile are loaded while the current
// tile's K/V rows are in flight.
template <int DT, int G, bool P1, int U>
__global__ __launch_bounds__(512) void decode_kernel(DecodeArgs a) {
  constexpr int kTile = 4 * U;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int waves = blockDim.x >> 6;
  const int h = blockIdx.y * waves + wave;  // kv head
  const int wg = blockIdx.x;
  if (wg >= a.ints[0] || h >= a.num_kv_heads) return;  // graph plans launch a fixed capacity
  const int item_end = a.ints[a.o_wg + wg + 1];
  for (int item = a.ints[a.o_wg + wg]; item < item_end; ++item) {
  const int4 w = reinterpret_cast<const int4*>(a.ints + a.o_work)[item];
  const int req = w.x, beg = w.y, end = w.z, pslot = w.w;
  const int grp = lane >> 4, sub = lane & 15;

  uint4 qv[G];
#pragma unroll
  for (int gi = 0; gi < G; ++gi)
    qv[gi] = ld128(a.q + req * a.q_stride_n + (h * G + gi) * a.q_stride_h + sub * 8);
  const int32_t* pages = a.indices + a.ints[a.o_indptr + req];
  wait_vmem_loads();
  const uint32_t row_elems = static_cast<uint32_t>(a.num_kv_heads) * kHeadDim;
  const uint16_t* kbase = a.k_cache + h * kHeadDim + sub * 8;
  const uint16_t* vbase = a.v_cache + h * kHeadDim + sub * 8;

  float m[G], l[G], o[G][8];
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    m[gi] = -1e30f;
    l[gi] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[gi][i] = 0.f;
  }

  uint64_t off[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int t = min(beg + 4 * u + grp, end - 1);
    off[u] = slot_offset<P1>(pages, t, a.page_size, row_elems);
  }
  for (int t0 = beg; t0 < end; t0 += kTile) {
    uint4 kr[U], vr[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      kr[u] = ld128(kbase + off[u]);
      vr[u] = ld128(vbase + off[u]);
      ok[u] = t0 + 4 * u + grp < end;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {  // next tile's slots, clamped into the chunk
      const int t = min(t0 + kTile + 4 * u + grp, end - 1);
      off[u] = slot_offset<P1>(pages, t, a.page_size, row_elems);
    }
    consume<DT, G, U>(qv, kr, vr, ok, a.scale_log2, m, l, o);
  }

  // Combine the four 16-lane groups of the wave (each saw a token subset).
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    float mx = fmaxf(m[gi], __shfl_xor(m[gi], 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float f = __builtin_amdgcn_exp2f(m[gi] - mx);
    float lv = l[gi] * f;
    lv += __shfl_xor(lv, 16);
    lv += __shfl_xor(lv, 32);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float x = o[gi][i] * f;
      x += __shfl_xor(x, 16);
      x += __shfl_xor(x, 32);
      o[gi][i] = x / lv;
    }
    m[gi] = mx;
    l[gi] = lv;
  }
  if (grp != 0) continue;
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    const int qh = h * G + gi;
    if (pslot < 0) {
      st128(a.out + req * a.out_stride_n + qh * a.out_stride_h + sub * 8, pack8<DT>(o[gi]));
    } else {
      float* dst =
          a.partial_o + (static_cast<int64_t>(pslot) * a.num_q_heads + qh) * kHeadDim + sub * 8;
      *reinterpret_cast<float4*>(dst) = make_float4(o[gi][0], o[gi][1], o[gi][2], o[gi][3]);
      *reinterpret_cast<float4*>(dst + 4) = make_float4(o[gi][4], o[gi][5], o[gi][6], o[gi][7]);
      if (sub == 0)  // log2-sum-exp of the chunk (v_log_f32 is log2)
        a.partial_lse[static_cast<int64_t>(pslot) * a.num_q_heads + qh] =
            m[gi] + __builtin_amdgcn_logf(l[gi]);
    }
  }
}  // item loop
}

// An item's page entries [0, n) -> LDS by direct copies (4 bytes per lane; lanes past
// n read entry n - 1, so every read stays inside the item's pages; the writes past n
// stay inside the entries array, whose size is a multiple of 64).
template <int W>
__device__ __forceinline__ void stage_entries(const int32_t* pages, int n, uint32_t lds,
                                              int wave, int lane) {
  for (int base = wave * 64; base < n; base += W * 64)
    copy_dword_to_lds(pages + min(base + lane, n - 1), lds + base * 4);
}

// Start of a work item: its request, token range, partial slot and the index of its
// first page entry in `indices`.
struct ItemStart {
  int req, beg, end, pslot, page_base;
};

__device__ __forceinline__ ItemStart item_start(const DecodeArgs& a, int item) {
  const int4 wi = reinterpret_cast<const int4*>(a.ints + a.o_work)[item];
  return {wi.x, wi.y, wi.z, wi.w, a.ints[a.o_indptr + wi.x] + wi.y / a.page_size};
}

// A workgroup's start record (written by the planner and pack_page_metadata), read with
// uniform loads from the constant address space so they become scalar loads that do
// not depend on each other: the first tile's copies need one round trip.
struct WgRecord {
  const __attribute__((address_space(4))) int32_t* p;
  __device__ WgRecord(const DecodeArgs& a, int wg)
      : p((const __attribute__((address_space(4))) int32_t*)(a.ints + a.o_wgrec) + kWgRec * wg) {}
  __device__ int item_begin() const { return p[0]; }
  __device__ int item_end() const { return p[1]; }
  __device__ ItemStart start() const { return {p[2], p[3], p[4], p[5], p[6]}; }
  __device__ uint32_t slot(int i) const { return static_cast<uint32_t>(p[kWgRecSlots + i]); }
};

// ---------------------------------------------------------------------------
// Decode with direct-to-LDS staging. One workgroup of W waves (one per kv head of
// its head slice) per CU; the grid is the balanced split-KV schedule, so every
// workgroup streams the same number of tokens. For each of its work items the
// workgroup copies the item's page entries to LDS, then streams T-token tiles of
// the K and V rows (W * 256 contiguous bytes per token and cache) through an
// S-deep LDS ring with global_load_lds_dwordx4: the copies need no registers and
// run S-1 tiles ahead of the math, and a page of P >= 4 tokens is read as long
// contiguous runs. Wave w computes kv head w of the slice from LDS exactly as
// decode_kernel does from registers.
// ---------------------------------------------------------------------------
template <int DT, int G, int W, int T, int S>
__global__ __launch_bounds__(64 * W, 1) void decode_dma_kernel(DecodeArgs a) {
  constexpr int kRow = W * 256;                 // bytes of one token's slice (K or V)
  constexpr int kHalf = T * kRow;               // K (or V) bytes of one tile
  constexpr int kStage = 2 * kHalf;
  constexpr int kCopies = 2 * kHalf / 1024;     // 1 KiB copies per tile
  constexpr int kPerWave = kCopies / W;
  constexpr int U = T / 4;                      // tokens per 16-lane group per tile
  static_assert(kRow >= 1024 && kRow % 1024 == 0, "a copy covers part of one token row");
  static_assert(kCopies % W == 0 && U % 2 == 0, "tile shape");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[S * kStage];
  __shared__ int32_t entries[kDmaMaxEntries];

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int grp = lane >> 4, sub = lane & 15;
  const int h = blockIdx.y * W + wave;  // kv head
  const int wg = blockIdx.x;
  if (wg >= a.ints[0]) return;  // graph plans launch a fixed capacity
  if (a.num_kv_heads < 0) {  // the copies are invisible to the compiler
    lds[threadIdx.x] = 0;
    entries[threadIdx.x] = 0;
  }
  const uint32_t lds_base = lds_address(lds);
  const uint32_t entries_lds = lds_address(entries);
  const uint32_t row_elems = static_cast<uint32_t>(a.num_kv_heads) * kHeadDim;
  const uint16_t* kslice = a.k_cache + blockIdx.y * W * kHeadDim;
  const uint16_t* vslice = a.v_cache + blockIdx.y * W * kHeadDim;
  const WgRecord rec(a, wg);
  const int item_begin = rec.item_begin(), item_end = rec.item_end();

  for (int item = item_begin; item < item_end; ++item) {
    // The workgroup's first item comes from its start record, whose slots let the first
    // tile's copies issue before the page entries are staged.
    const bool first = item == item_begin;
    const ItemStart is = first ? rec.start() : item_start(a, item);
    const int req = is.req, beg = is.beg, end = is.end, pslot = is.pslot;
    const int first_page = beg / a.page_size;
    const int n_entries = (end - 1) / a.page_size - first_page + 1;
    const int32_t* pages = a.indices + is.page_base;
    const int n_tiles = (end - beg + T - 1) / T;
    // Copy c of a tile: half c / (kCopies / 2) (K, V), token (c % (kCopies / 2)) * 1024 /
    // kRow of the tile, byte (c * 1024) % kRow of its row; the token is wave-uniform.
    // Tile 0 of the first item reads its slots from the start record, every other tile
    // from the page entries staged in LDS.
    auto issue = [&](int t, int stage, bool from_record) {
#pragma unroll
      for (int j = 0; j < kPerWave; ++j) {
        const int c = wave * kPerWave + j;
        const int half = c / (kCopies / 2);
        const int r = c % (kCopies / 2);
        const int tok = min(beg + t * T + (r * 1024) / kRow, end - 1);
        uint32_t slot;
        if (from_record) {
          slot = rec.slot(tok - beg);
        } else {
          const int e = entries[tok / a.page_size - first_page];
          slot = static_cast<uint32_t>(e) * static_cast<uint32_t>(a.page_size) +
                 static_cast<uint32_t>(tok % a.page_size);
        }
        const uint16_t* src = (half ? vslice : kslice) + static_cast<uint64_t>(slot) * row_elems +
                              ((r * 1024) % kRow) / 2 + lane * 8;
        copy_to_lds(src, lds_base + stage * kStage + half * kHalf + r * 1024);
      }
    };
    // Page entries of tokens [beg, end) -> LDS (the previous item's readers are done),
    // then the query rows. The first item's tile 0 issues right behind them; the loop's
    // first wait (vmcnt 0) covers entries, queries and that tile, and its barrier makes
    // the entries visible before tile 1 is issued.
    if (!first) __syncthreads();
    stage_entries<W>(pages, n_entries, entries_lds, wave, lane);
    uint4 qv[G];
#pragma unroll
    for (int gi = 0; gi < G; ++gi)
      qv[gi] = ld128(a.q + req * a.q_stride_n + (h * G + gi) * a.q_stride_h + sub * 8);
    if (first) issue(0, 0, true);  // nothing has used the ring yet
    if (!first || S > 2) {
      wait_vmem_loads();
      __syncthreads();
    }

    float m[G], l[G], o[G][8];
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      m[gi] = -1e30f;
      l[gi] = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[gi][i] = 0.f;
    }
    for (int st = first ? 1 : 0; st < S - 1; ++st)
      if (st < n_tiles) issue(st, st, false);
    for (int t = 0; t < n_tiles; ++t) {
      wait_tiles_ahead<kPerWave, S - 2>(min(S - 2, n_tiles - 1 - t));
      __syncthreads();
      if (t + S - 1 < n_tiles) issue(t + S - 1, (t + S - 1) % S, false);
      const uint8_t* sb = lds + (t % S) * kStage + wave * 256 + sub * 16;
      uint4 kr[U], vr[U];
      bool ok[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int tt = 4 * u + grp;
        kr[u] = *reinterpret_cast<const uint4*>(sb + tt * kRow);
        vr[u] = *reinterpret_cast<const uint4*>(sb + kHalf + tt * kRow);
        ok[u] = beg + t * T + tt < end;
      }
      consume<DT, G, U>(qv, kr, vr, ok, a.scale_log2, m, l, o);
    }

#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      float mx = fmaxf(m[gi], __shfl_xor(m[gi], 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float f = __builtin_amdgcn_exp2f(m[gi] - mx);
      float lv = l[gi] * f;
      lv += __shfl_xor(lv, 16);
      lv += __shfl_xor(lv, 32);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float x = o[gi][i] * f;
        x += __shfl_xor(x, 16);
        x += __shfl_xor(x, 32);
        o[gi][i] = x / lv;
      }
      m[gi] = mx;
      l[gi] = lv;
    }
    if (grp == 0) {
#pragma unroll
      for (int gi = 0; gi < G; ++gi) {
        const int qh = h * G + gi;
        if (pslot < 0) {
          st128(a.out + req * a.out_stride_n + qh * a.out_stride_h + sub * 8, pack8<DT>(o[gi]));
        } else {
          float* dst = a.partial_o +
                       (static_cast<int64_t>(pslot) * a.num_q_heads + qh) * kHeadDim + sub * 8;
          *reinterpret_cast<float4*>(dst) = make_float4(o[gi][0], o[gi][1], o[gi][2], o[gi][3]);
          *reinterpret_cast<float4*>(dst + 4) =
              make_float4(o[gi][4], o[gi][5], o[gi][6], o[gi][7]);
          if (sub == 0)
            a.partial_lse[static_cast<int64_t>(pslot) * a.num_q_heads + qh] =
                m[gi] + __builtin_amdgcn_logf(l[gi]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// decode_mma_kernel: decode_dma_kernel's copy pipeline with the math on the matrix
// cores, for GQA groups of 4..16 q heads per kv head (Qwen3-8B: 4). Per 16-token tile,
// wave w (kv head w of the slice) computes
//   S = K Q^T   with v_mfma_f32_16x16x32 (A = 16 K rows, B = the group's q heads as
//               columns; columns past the group are zero), 4 MFMAs over d = 128;
//   P = 2^(S scale - m) per column (online softmax; the S accumulator already holds each
//               lane's 4 tokens of one column, the B layout of the next product);
//   O^T += V^T P^T with v_mfma_f32_16x16x16, 8 MFMAs (one per 16 dims), the V^T operand
//               read transposed from the row-major V tile with ds_read_b64_tr_b16.
// The copies place 16-byte chunk c of a head's 256 bytes at position c ^ (token & 15) of
// its token row, so the 16 rows an MFMA operand read touches land in distinct banks.
// ---------------------------------------------------------------------------
typedef __bf16 mma_bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 mma_bf16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 mma_f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 mma_f16x4_t __attribute__((ext_vector_type(4)));
typedef float mma_floatx4 __attribute__((ext_vector_type(4)));
typedef short mma_v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) mma_v4i16_t mma_lds_v4i16;

template <int DT>
__device__ __forceinline__ mma_floatx4 mma_16x16x32(const uint4& a, const uint4& b,
                                                    mma_floatx4 c) {
  if constexpr (DT == 0)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(mma_bf16x8_t, a),
                                                   __builtin_bit_cast(mma_bf16x8_t, b), c, 0, 0,
                                                   0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(mma_f16x8_t, a),
                                                  __builtin_bit_cast(mma_f16x8_t, b), c, 0, 0, 0);
}

template <int DT>
__device__ __forceinline__ mma_floatx4 mma_16x16x16(const uint2& a, const uint2& b,
                                                    mma_floatx4 c) {
  if constexpr (DT == 0)
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(mma_v4i16_t, a),
                                                     __builtin_bit_cast(mma_v4i16_t, b), c, 0,
                                                     0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(mma_f16x4_t, a),
                                                 __builtin_bit_cast(mma_f16x4_t, b), c, 0, 0, 0);
}

template <int DT, int G, int W, int S>
__global__ __launch_bounds__(64 * W, 1) void decode_mma_kernel(DecodeArgs a) {
  constexpr int T = 16;                         // tokens per tile = the MFMAs' 16 rows
  constexpr int kRow = W * 256;                 // bytes of one token's slice (K or V)
  constexpr int kHalf = T * kRow;               // K (or V) bytes of one tile
  constexpr int kStage = 2 * kHalf;
  constexpr int kCopies = 2 * kHalf / 1024;     // 1 KiB copies per tile
  constexpr int kPerWave = kCopies / W;
  static_assert(G >= 2 && G <= 16, "the q heads of a group are the MFMA columns");
  static_assert(kRow >= 1024 && kRow % 1024 == 0 && kCopies % W == 0, "tile shape");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[S * kStage];
  __shared__ int32_t entries[kDmaMaxEntries];

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;   // MFMA column (q head of the group) / operand row
  const int quad = lane >> 4;  // 16-lane group
  const int h = blockIdx.y * W + wave;  // kv head
  const int wg = blockIdx.x;
  if (wg >= a.ints[0]) return;  // graph plans launch a fixed capacity
  if (a.num_kv_heads < 0) {  // the copies are invisible to the compiler
    lds[threadIdx.x] = 0;
    entries[threadIdx.x] = 0;
  }
  const uint32_t lds_base = lds_address(lds);
  const uint32_t entries_lds = lds_address(entries);
  const uint32_t row_elems = static_cast<uint32_t>(a.num_kv_heads) * kHeadDim;
  const uint16_t* kslice = a.k_cache + blockIdx.y * W * kHeadDim;
  const uint16_t* vslice = a.v_cache + blockIdx.y * W * kHeadDim;
  const WgRecord rec(a, wg);
  const int item_begin = rec.item_begin(), item_end = rec.item_end();

  // Read offsets within a stage for this wave's head (token-independent parts).
  const int head_off = wave * 256;

  for (int item = item_begin; item < item_end; ++item) {
    // The first item comes from the start record (see decode_dma_kernel).
    const bool first = item == item_begin;
    const ItemStart is = first ? rec.start() : item_start(a, item);
    const int req = is.req, beg = is.beg, end = is.end, pslot = is.pslot;
    const int first_page = beg / a.page_size;
    const int n_entries = (end - 1) / a.page_size - first_page + 1;
    const int32_t* pages = a.indices + is.page_base;
    const int n_tiles = (end - beg + T - 1) / T;
    // Copy c of a tile: half c / (kCopies / 2) (K, V), token (c % (kCopies / 2)) * 1024 /
    // kRow of the tile, byte (c * 1024) % kRow of its row; the token is wave-uniform.
    // Lane i fetches the chunk that belongs at position i: chunk (i ^ (token & 15)) of
    // the same head. Tile 0 of the first item reads its slots from the start record.
    auto issue = [&](int t, int stage, bool from_record) {
#pragma unroll
      for (int j = 0; j < kPerWave; ++j) {
        const int c = wave * kPerWave + j;
        const int half = c / (kCopies / 2);
        const int r = c % (kCopies / 2);
        const int tile_tok = (r * 1024) / kRow;
        const int tok = min(beg + t * T + tile_tok, end - 1);
        uint32_t slot;
        if (from_record) {
          slot = rec.slot(tok - beg);
        } else {
          const int e = entries[tok / a.page_size - first_page];
          slot = static_cast<uint32_t>(e) * static_cast<uint32_t>(a.page_size) +
                 static_cast<uint32_t>(tok % a.page_size);
        }
        const int chunk = ((r * 1024) % kRow) / 16 + lane;  // position within the row
        const int src_chunk = (chunk & ~15) | ((chunk & 15) ^ (tile_tok & 15));
        const uint16_t* src =
            (half ? vslice : kslice) + static_cast<uint64_t>(slot) * row_elems + src_chunk * 8;
        copy_to_lds(src, lds_base + stage * kStage + half * kHalf + r * 1024);
      }
    };
    if (!first) __syncthreads();
    stage_entries<W>(pages, n_entries, entries_lds, wave, lane);
    // Q^T as the B operand: lane holds q head (h G + col) dims 32 kk + 8 quad .. + 8;
    // columns past the group are zero.
    uint4 qb[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      qb[kk] = col < G ? ld128(a.q + req * a.q_stride_n + (h * G + col) * a.q_stride_h +
                               32 * kk + 8 * quad)
                       : make_uint4(0, 0, 0, 0);
    }
    if (first) issue(0, 0, true);  // nothing has used the ring yet
    if (!first || S > 2) {
      wait_vmem_loads();
      __syncthreads();
    }


    mma_floatx4 o[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) o[b] = mma_floatx4{0.f, 0.f, 0.f, 0.f};
    float m = -1e30f, l = 0.f;  // of column `col`; m is the same in the 4 lane groups

    for (int st = first ? 1 : 0; st < S - 1; ++st)
      if (st < n_tiles) issue(st, st, false);
    for (int t = 0; t < n_tiles; ++t) {
      wait_tiles_ahead<kPerWave, S - 2>(min(S - 2, n_tiles - 1 - t));
      __syncthreads();
      if (t + S - 1 < n_tiles) issue(t + S - 1, (t + S - 1) % S, false);
      const uint8_t* kb = lds + (t % S) * kStage + head_off;
      const uint8_t* vb = kb + kHalf;
      // S = K Q^T: lane reads token `col`, chunk 4 kk + quad (swizzled).
      mma_floatx4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const uint4 kf = *reinterpret_cast<const uint4*>(kb + col * kRow +
                                                          (((4 * kk + quad) ^ col) * 16));
        sc = mma_16x16x32<DT>(kf, qb[kk], sc);
      }
      // V^T operands (transposed reads): block b, lane p of group quad addresses token
      // 4 quad + p / 4, dims 16 b + 4 (p % 4) .. + 3.
      uint2 vf[8];
      {
        const int vt = 4 * quad + (col >> 2);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
          const int chunk = 2 * b + ((col & 3) >> 1);
          lds_u8* vp = (lds_u8*)vb + vt * kRow + ((chunk ^ vt) * 16) + 8 * (col & 1);
          vf[b] = __builtin_bit_cast(
              uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((mma_lds_v4i16*)vp));
        }
      }
      // Lane holds S[token 4 quad + i][col]; tokens past the item are masked.
      float s[4];
      float mx = m;
      const int tok0 = beg + t * T + 4 * quad;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s[i] = tok0 + i < end ? sc[i] * a.scale_log2 : -INFINITY;
        mx = fmaxf(mx, s[i]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float corr = __builtin_amdgcn_exp2f(m - mx);
      m = mx;
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(s[i] - mx);
      l = l * corr + ((p[0] + p[1]) + (p[2] + p[3]));
      const uint2 pb = make_uint2(Elem<DT>::pack2(p[0], p[1]), Elem<DT>::pack2(p[2], p[3]));
#pragma unroll
      for (int b = 0; b < 8; ++b) {
#pragma unroll
        for (int i = 0; i < 4; ++i) o[b][i] *= corr;
        o[b] = mma_16x16x16<DT>(vf[b], pb, o[b]);
      }
    }

    // Column totals: l summed over the 4 lane groups (m is already common).
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    if (col < G) {
      const int qh = h * G + col;
      const float inv = 1.f / l;
      // Lane holds O^T[16 b + 4 quad + i][col].
      if (pslot < 0) {
        uint16_t* dst = a.out + req * a.out_stride_n + qh * a.out_stride_h + 4 * quad;
#pragma unroll
        for (int b = 0; b < 8; ++b)
          *reinterpret_cast<uint2*>(dst + 16 * b) =
              make_uint2(Elem<DT>::pack2(o[b][0] * inv, o[b][1] * inv),
                         Elem<DT>::pack2(o[b][2] * inv, o[b][3] * inv));
      } else {
        float* dst = a.partial_o +
                     (static_cast<int64_t>(pslot) * a.num_q_heads + qh) * kHeadDim + 4 * quad;
#pragma unroll
        for (int b = 0; b < 8; ++b)
          *reinterpret_cast<float4*>(dst + 16 * b) =
              make_float4(o[b][0] * inv, o[b][1] * inv, o[b][2] * inv, o[b][3] * inv);
        if (quad == 0)
          a.partial_lse[static_cast<int64_t>(pslot) * a.num_q_heads + qh] =
              m + __builtin_amdgcn_logf(l);
      }
    }
  }
}

// Split-KV merge: one wave per (request, q head), two dims per lane. Chunks are
// combined with a running log2-sum-exp; the chunk loop is unrolled so the
// partial loads of several chunks are in flight together.
template <int DT>
__global__ __launch_bounds__(256) void merge_kernel(DecodeArgs a, int32_t rows) {
  const int req = blockIdx.x;
  const int qh = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (req >= rows || qh >= a.num_q_heads) return;
  const int first = a.ints[a.o_merge + 2 * req];
  const int count = a.ints[a.o_merge + 2 * req + 1];
  if (count <= 1) return;
  constexpr int kUnroll = 8;
  float mx = -INFINITY, den = 0.f, acc0 = 0.f, acc1 = 0.f;
  for (int c0 = 0; c0 < count; c0 += kUnroll) {
    float lse[kUnroll];
    float2 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int c = min(c0 + u, count - 1);
      const int64_t p = static_cast<int64_t>(first + c) * a.num_q_heads + qh;
      lse[u] = c0 + u < count ? a.partial_lse[p] : -INFINITY;
      v[u] = *reinterpret_cast<const float2*>(a.partial_o + p * kHeadDim + lane * 2);
    }
    float m_new = mx;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) m_new = fmaxf(m_new, lse[u]);
    const float corr = __builtin_amdgcn_exp2f(mx - m_new);
    den *= corr;
    acc0 *= corr;
    acc1 *= corr;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const float wgt = __builtin_amdgcn_exp2f(lse[u] - m_new);
      den += wgt;
      acc0 = fmaf(wgt, v[u].x, acc0);
      acc1 = fmaf(wgt, v[u].y, acc1);
    }
    mx = m_new;
  }
  const uint32_t packed = static_cast<uint32_t>(Elem<DT>::from_float(acc0 / den)) |
                          (static_cast<uint32_t>(Elem<DT>::from_float(acc1 / den)) << 16);
  *reinterpret_cast<uint32_t*>(a.out + req * a.out_stride_n + qh * a.out_stride_h + lane * 2) =
      packed;
}

// Tokens per 16-lane group per loop trip. Override with MI355X_DECODE_U
// (2, 4 or 8; tuning knob, read once).
int tokens_per_group() {
  static const int value = [] {
    const char* env = std::getenv("MI355X_DECODE_U");
    const int v = env ? std::atoi(env) : 0;
    return (v == 2 || v == 4 || v == 8) ? v : kTokensPerLaneGroup;
  }();
  return value;
}

template <int DT, int G>
void launch_decode(const DecodeArgs& a, dim3 grid, int waves, bool p1, hipStream_t s) {
  const dim3 block(waves * kWave);
  const int u = tokens_per_group();
#define MI355X_DECODE_LAUNCH(P, UU) decode_kernel<DT, G, P, UU><<<grid, block, 0, s>>>(a)
  if (p1) {
    if (u == 2) MI355X_DECODE_LAUNCH(true, 2);
    else if (u == 8) MI355X_DECODE_LAUNCH(true, 8);
    else MI355X_DECODE_LAUNCH(true, 4);
  } else {
    if (u == 2) MI355X_DECODE_LAUNCH(false, 2);
    else if (u == 8) MI355X_DECODE_LAUNCH(false, 8);
    else MI355X_DECODE_LAUNCH(false, 4);
  }
#undef MI355X_DECODE_LAUNCH
}

template <int DT>
bool dispatch_group(const DecodeArgs& a, int group, dim3 grid, int waves, bool p1,
                    hipStream_t s) {
  switch (group) {
    case 1: launch_decode<DT, 1>(a, grid, waves, p1, s); return true;
    case 2: launch_decode<DT, 2>(a, grid, waves, p1, s); return true;
    case 4: launch_decode<DT, 4>(a, grid, waves, p1, s); return true;
    case 8: launch_decode<DT, 8>(a, grid, waves, p1, s); return true;
    default: return false;
  }
}

// Matrix-core math for GQA groups of 4 or more (MI355X_DECODE_MMA=0 turns it off; tuning
// knob, read once).
bool mma_enabled() {
  static const bool on = [] {
    const char* env = std::getenv("MI355X_DECODE_MMA");
    return !(env && std::strcmp(env, "0") == 0);
  }();
  return on;
}

template <int DT, int G>
void launch_dma(const DecodeArgs& a, dim3 grid, int waves, hipStream_t s) {
  if constexpr (G >= 4) {
    if (mma_enabled()) {
      if (waves == 8)
        decode_mma_kernel<DT, G, 8, kDmaStages><<<grid, dim3(8 * kWave), 0, s>>>(a);
      else
        decode_mma_kernel<DT, G, 4, kDmaStages><<<grid, dim3(4 * kWave), 0, s>>>(a);
      return;
    }
  }
  if (waves == 8)
    decode_dma_kernel<DT, G, 8, kDmaTile, kDmaStages><<<grid, dim3(8 * kWave), 0, s>>>(a);
  else
    decode_dma_kernel<DT, G, 4, kDmaTile, kDmaStages><<<grid, dim3(4 * kWave), 0, s>>>(a);
}

template <int DT>
bool dispatch_dma(const DecodeArgs& a, int group, dim3 grid, int waves, hipStream_t s) {
  switch (group) {
    case 1: launch_dma<DT, 1>(a, grid, waves, s); return true;
    case 2: launch_dma<DT, 2>(a, grid, waves, s); return true;
    case 4: launch_dma<DT, 4>(a, grid, waves, s); return true;
    case 8: launch_dma<DT, 8>(a, grid, waves, s); return true;
    default: return false;
  }
}

}  // namespace
}  // namespace mi355x

using namespace mi355x;

extern "C" int64_t mi355x_decode_schedule(const int32_t* lengths, int64_t batch, int64_t cus,
                                          int64_t num_kv_heads, int32_t* work,
                                          int64_t work_capacity, int32_t* merge,
                                          int64_t* chunk_tokens) {
  if (!lengths || batch < 0 || cus <= 0 || num_kv_heads <= 0 || !work || !merge || !chunk_tokens)
    return -1;
  for (int64_t r = 0; r < batch; ++r)
    if (lengths[r] <= 0) return -1;
  // The host-only view: page size 1 and no cap on item length.
  const LaunchShape shape = launch_shape(cus, num_kv_heads, 1);
  return schedule(lengths, batch, shape.workgroups, std::numeric_limits<int32_t>::max(),
                  shape.tile, work,
                  work_capacity, merge, chunk_tokens);
}

extern "C" int64_t mi355x_decode_items_capacity(int64_t rows, int64_t cus, int64_t num_kv_heads) {
  if (rows < 0 || cus <= 0 || num_kv_heads <= 0) return -1;
  return launch_shape(cus, num_kv_heads, 1).wg_capacity + rows;
}

extern "C" void* mi355x_decode_prepare(void* existing, const int32_t* block_table,
                                       int64_t batch, int64_t columns, int64_t table_stride,
                                       const int32_t* seq_lens, int64_t num_q_heads,
                                       int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                                       int64_t dtype, bool graph, const int32_t* host_lengths,
                                       int64_t host_rows, void* stream) {
  auto s = static_cast<hipStream_t>(stream);
  std::unique_ptr<DecodePlan> created;
  DecodePlan* plan = static_cast<DecodePlan*>(existing);
  try {
    if (!block_table || !seq_lens || batch <= 0 || columns <= 0 || table_stride < columns) {
      set_error("invalid decode block table or lengths");
      return nullptr;
    }
    if (num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 ||
        head_dim != kHeadDim || page_size <= 0 || (dtype != 0 && dtype != 1)) {
      set_error("unsupported decode attention configuration");
      return nullptr;
    }
    const int64_t group = num_q_heads / num_kv_heads;
    if (group != 1 && group != 2 && group != 4 && group != 8) {
      set_error("decode attention supports 1, 2, 4 or 8 query heads per kv head");
      return nullptr;
    }
    int device = 0;
    hipError_t st = hipGetDevice(&device);
    if (st != hipSuccess) {
      hip_error(st, "hipGetDevice");
      return nullptr;
    }
    if (plan && (plan->device != device || plan->num_q_heads != num_q_heads ||
                 plan->num_kv_heads != num_kv_heads || plan->head_dim != head_dim ||
                 plan->page_size != page_size || plan->dtype != dtype || plan->graph != graph ||
                 (graph && (plan->graph_columns != columns || plan->graph_rows != batch)))) {
      set_error("decode workspace geometry changed");
      return nullptr;
    }
    if (!plan) {
      created = std::make_unique<DecodePlan>();
      plan = created.get();
      plan->device = device;
      int cus = 0;
      st = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
      if (st != hipSuccess) {
        hip_error(st, "hipDeviceGetAttribute");
        return nullptr;
      }
      plan->cus = std::max(cus, 1);
      plan->num_q_heads = num_q_heads;
      plan->num_kv_heads = num_kv_heads;
      plan->head_dim = head_dim;
      plan->page_size = page_size;
      plan->dtype = dtype;
      plan->graph = graph;
      plan->graph_rows = batch;
      plan->graph_columns = columns;
      st = hipEventCreateWithFlags(&plan->upload_done, hipEventDisableTiming);
      if (st != hipSuccess) {
        hip_error(st, "hipEventCreate");
        return nullptr;
      }
    }

    // Host lengths: the scheduler's snapshot when given, else one D2H read.
    plan->host_lengths.resize(batch);
    if (host_lengths) {
      if (host_rows != batch) {
        set_error("invalid host decode metadata");
        return nullptr;
      }
      std::memcpy(plan->host_lengths.data(), host_lengths, batch * sizeof(int32_t));
    } else {
      st = hipMemcpyAsync(plan->host_lengths.data(), seq_lens, batch * sizeof(int32_t),
                          hipMemcpyDeviceToHost, s);
      if (st == hipSuccess) st = hipStreamSynchronize(s);
      if (st != hipSuccess) {
        hip_error(st, "decode length readback");
        return nullptr;
      }
    }
    int64_t total_pages = 0;
    for (int64_t r = 0; r < batch; ++r) {
      const int64_t len = plan->host_lengths[r];
      if (len <= 0 || len > columns * page_size) {
        set_error("host cache length exceeds block table capacity");
        return nullptr;
      }
      total_pages += (len + page_size - 1) / page_size;
      if (total_pages > std::numeric_limits<int32_t>::max()) {
        set_error("page indptr overflow");
        return nullptr;
      }
    }

    const LaunchShape shape = launch_shape(plan->cus, num_kv_heads, page_size);
    const int64_t items_cap = items_capacity_for(shape, batch, columns * page_size);
    const int64_t wg_cap = shape.wg_capacity;
    const IntLayout layout = IntLayout::make(batch, items_cap, wg_cap);
    const size_t int_bytes = layout.total * sizeof(int32_t);
    const size_t idx_bytes = static_cast<size_t>(batch) * columns * sizeof(int32_t);
    const size_t part_o_bytes = static_cast<size_t>(items_cap) * num_q_heads * kHeadDim * 4;
    const size_t part_lse_bytes = static_cast<size_t>(items_cap) * num_q_heads * 4;
    const size_t last_bytes = static_cast<size_t>(batch) * sizeof(int32_t);
    if (graph && !created &&
        (int_bytes > plan->ints.capacity || idx_bytes > plan->indices.capacity ||
         part_o_bytes > plan->partial_o.capacity || last_bytes > plan->last_len.capacity)) {
      set_error("graph decode metadata capacity exceeded");
      return nullptr;
    }
    // The pinned staging buffer may still be feeding the previous upload.
    st = hipEventSynchronize(plan->upload_done);
    if (st != hipSuccess) {
      hip_error(st, "decode upload fence");
      return nullptr;
    }
    if ((st = plan->ints.reserve(int_bytes, plan->allocations)) != hipSuccess ||
        (st = plan->indices.reserve(idx_bytes, plan->allocations)) != hipSuccess ||
        (st = plan->last_len.reserve(last_bytes, plan->allocations)) != hipSuccess ||
        (st = plan->partial_o.reserve(part_o_bytes, plan->allocations)) != hipSuccess ||
        (st = plan->partial_lse.reserve(part_lse_bytes, plan->allocations)) != hipSuccess ||
        (st = plan->staging.reserve(int_bytes, plan->allocations)) != hipSuccess) {
      hip_error(st, "decode workspace allocation");
      return nullptr;
    }
    int32_t* host = static_cast<int32_t*>(plan->staging.ptr);
    // Everything before the start records starts at zero; the records of the workgroups
    // launched are written in full below (those past them are never read).
    std::memset(host, 0, layout.o_wgrec * sizeof(int32_t));
    int32_t* indptr = host + layout.o_indptr;
    indptr[0] = 0;
    for (int64_t r = 0; r < batch; ++r)
      indptr[r + 1] = indptr[r] + static_cast<int32_t>(
                                      (plan->host_lengths[r] + page_size - 1) / page_size);
    int64_t chunk = 0, wgs = 0;
    const int64_t items = schedule(plan->host_lengths.data(), batch, shape.workgroups,
                                   shape.max_item, shape.tile, host + layout.o_work, items_cap,
                                   host + layout.o_merge, &chunk, host + layout.o_wg, wg_cap, &wgs);
    if (items < 0) {
      set_error("decode work list exceeds its capacity");
      return nullptr;
    }
    host[0] = static_cast<int32_t>(wgs);
    host[1] = static_cast<int32_t>(items);
    // Start records: the first item of each workgroup and the page-entry index of its
    // first token (pack_page_metadata fills the slots from the block table).
    for (int64_t w = 0; w < wgs; ++w) {
      int32_t* rec = host + layout.o_wgrec + kWgRec * w;
      const int32_t* first = host + layout.o_wg;
      std::memset(rec, 0, kWgRecSlots * sizeof(int32_t));
      rec[0] = first[w];
      rec[1] = first[w + 1];
      if (rec[0] < rec[1]) {
        const int32_t* wi = host + layout.o_work + 4 * static_cast<int64_t>(rec[0]);
        rec[2] = wi[0];
        rec[3] = wi[1];
        rec[4] = wi[2];
        rec[5] = wi[3];
        rec[6] = indptr[wi[0]] + wi[1] / static_cast<int32_t>(page_size);
      }
    }
    const size_t upload_bytes = (layout.o_wgrec + kWgRec * wgs) * sizeof(int32_t);
    st = hipMemcpyAsync(plan->ints.ptr, host, upload_bytes, hipMemcpyHostToDevice, s);
    if (st != hipSuccess) {
      hip_error(st, "decode metadata upload");
      return nullptr;
    }
    pack_page_metadata<<<dim3(static_cast<uint32_t>(std::max(batch, wgs))), dim3(256), 0, s>>>(
        block_table, seq_lens, static_cast<const int32_t*>(plan->ints.ptr) + layout.o_indptr,
        static_cast<int32_t*>(plan->indices.ptr), static_cast<int32_t*>(plan->last_len.ptr),
        table_stride, static_cast<int32_t>(page_size),
        static_cast<int32_t*>(plan->ints.ptr) + layout.o_wgrec, static_cast<int32_t>(wgs),
        static_cast<int32_t>(batch));
    if (const char* err = launch_status("pack_page_metadata")) {
      (void)err;
      return nullptr;
    }
    st = hipEventRecord(plan->upload_done, s);
    if (st != hipSuccess) {
      hip_error(st, "decode upload event");
      return nullptr;
    }
    plan->batch = batch;
    plan->total_pages = total_pages;
    plan->num_items = items;
    plan->chunk_tokens = chunk;
    plan->items_capacity = items_cap;
    plan->num_wgs = wgs;
    plan->wg_capacity = wg_cap;
    plan->layout = layout;
    created.release();
    return plan;
  } catch (const std::exception& e) {
    set_error(e.what());
    return nullptr;
  }
}

extern "C" void mi355x_decode_plan_drop(void* plan) {
  delete static_cast<DecodePlan*>(plan);
}

extern "C" uint64_t mi355x_decode_workspace_allocations(const void* plan) {
  return plan ? static_cast<const DecodePlan*>(plan)->allocations : 0;
}

// Plan facts: [batch, total_pages, num_items, chunk_tokens, items_capacity, cus].
extern "C" const char* mi355x_decode_plan_info(const void* plan, int64_t* out6) {
  if (!plan || !out6) return set_error("mi355x_decode_plan_info: null argument");
  const auto* p = static_cast<const DecodePlan*>(plan);
  out6[0] = p->batch;
  out6[1] = p->total_pages;
  out6[2] = p->num_items;
  out6[3] = p->chunk_tokens;
  out6[4] = p->items_capacity;
  out6[5] = p->cus;
  return nullptr;
}

// Synchronous copy of the plan's page metadata and work list to host memory.
// Sizes: indptr batch+1, indices total_pages, last_len batch,
// work 4*num_items, merge 2*batch (any pointer may be NULL).
extern "C" const char* mi355x_decode_plan_read(const void* plan, int32_t* indptr,
                                               int32_t* indices, int32_t* last_len,
                                               int32_t* work, int32_t* merge, void* stream) {
  if (!plan) return set_error("mi355x_decode_plan_read: null plan");
  const auto* p = static_cast<const DecodePlan*>(plan);
  auto s = static_cast<hipStream_t>(stream);
  const int32_t* ints = static_cast<const int32_t*>(p->ints.ptr);
  hipError_t st = hipSuccess;
  auto copy = [&](void* dst, const void* src, size_t bytes) {
    if (dst && st == hipSuccess && bytes)
      st = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s);
  };
  copy(indptr, ints + p->layout.o_indptr, (p->batch + 1) * 4);
  copy(indices, p->indices.ptr, p->total_pages * 4);
  copy(last_len, p->last_len.ptr, p->batch * 4);
  copy(work, ints + p->layout.o_work, p->num_items * 16);
  copy(merge, ints + p->layout.o_merge, p->batch * 8);
  if (st == hipSuccess) st = hipStreamSynchronize(s);
  return st == hipSuccess ? nullptr : hip_error(st, "mi355x_decode_plan_read");
}

extern "C" const char* mi355x_decode_run(const void* plan_ptr, const void* q, int64_t q_stride_n,
                                         int64_t q_stride_h, const void* k_cache,
                                         const void* v_cache, void* out, int64_t out_stride_n,
                                         int64_t out_stride_h, int64_t batch, int64_t num_q_heads,
                                         int64_t num_kv_heads, int64_t page_size, int64_t dtype,
                                         void* stream) {
  if (!plan_ptr) return set_error("decode was not prepared");
  const auto& p = *static_cast<const DecodePlan*>(plan_ptr);
  if (!q || !k_cache || !v_cache || !out) return set_error("mi355x_decode_run: null pointer");
  if (num_q_heads != p.num_q_heads || num_kv_heads != p.num_kv_heads ||
      page_size != p.page_size || dtype != p.dtype || batch != p.batch)
    return set_error("decode tensors do not match the prepared batch");
  if (q_stride_h % 8 || q_stride_n % 8 || out_stride_h % 8 || out_stride_n % 8 ||
      !aligned(q, 16) || !aligned(out, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16))
    return set_error("decode requires 16-byte aligned rows");
  DecodeArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.q_stride_n = q_stride_n;
  a.q_stride_h = q_stride_h;
  a.k_cache = static_cast<const uint16_t*>(k_cache);
  a.v_cache = static_cast<const uint16_t*>(v_cache);
  a.out = static_cast<uint16_t*>(out);
  a.out_stride_n = out_stride_n;
  a.out_stride_h = out_stride_h;
  a.ints = static_cast<const int32_t*>(p.ints.ptr);
  a.o_indptr = static_cast<int32_t>(p.layout.o_indptr);
  a.o_work = static_cast<int32_t>(p.layout.o_work);
  a.o_merge = static_cast<int32_t>(p.layout.o_merge);
  a.o_wg = static_cast<int32_t>(p.layout.o_wg);
  a.o_wgrec = static_cast<int32_t>(p.layout.o_wgrec);
  a.indices = static_cast<const int32_t*>(p.indices.ptr);
  a.partial_o = static_cast<float*>(p.partial_o.ptr);
  a.partial_lse = static_cast<float*>(p.partial_lse.ptr);
  a.num_q_heads = static_cast<int32_t>(num_q_heads);
  a.num_kv_heads = static_cast<int32_t>(num_kv_heads);
  a.page_size = static_cast<int32_t>(page_size);
  a.scale_log2 = (1.0f / std::sqrt(static_cast<float>(kHeadDim))) * kLog2e;

  const LaunchShape shape = launch_shape(p.cus, num_kv_heads, page_size);
  const int waves = static_cast<int>(shape.waves);
  // Graph plans launch the fixed capacity; surplus workgroups exit at once.
  const int64_t grid_x = p.graph ? p.wg_capacity : p.num_wgs;
  const dim3 grid(static_cast<uint32_t>(grid_x), static_cast<uint32_t>(shape.grid_y));
  const int group = static_cast<int>(num_q_heads / num_kv_heads);
  auto s = static_cast<hipStream_t>(stream);
  const bool ok =
      shape.dma
          ? (dtype == 0 ? dispatch_dma<0>(a, group, grid, waves, s)
                        : dispatch_dma<1>(a, group, grid, waves, s))
          : (dtype == 0 ? dispatch_group<0>(a, group, grid, waves, page_size == 1, s)
                        : dispatch_group<1>(a, group, grid, waves, page_size == 1, s));
  if (!ok) return set_error("unsupported query group size");
  if (const char* err = launch_status("decode_kernel")) return err;
  if (p.graph || p.num_items > p.batch) {  // some request was split
    const dim3 mgrid(static_cast<uint32_t>(batch), static_cast<uint32_t>((num_q_heads + 3) / 4));
    if (dtype == 0)
      merge_kernel<0><<<mgrid, dim3(256), 0, s>>>(a, static_cast<int32_t>(batch));
    else
      merge_kernel<1><<<mgrid, dim3(256), 0, s>>>(a, static_cast<int32_t>(batch));
    return launch_status("merge_kernel");
  }
  return nullptr;
}
