// Decode-step projection GEMMs on gfx950: out[M, N] = x[M, K] . w[N, K]^T.
//
// Replaces the reference's `x.matmul(w.T)` (src/layers/linear.rs:5-7, cuBLAS through
// tch) for the decoder layer's QKV, o_proj and down projections when the batch is a
// decode batch (M <= 256 rows), the last two optionally fused with the residual RMSNorm
// that follows them, and the gate_up projection fused with SiLU x mul. Prefill-sized
// products and the lm_head stay on hipBLASLt, which runs them near the MFMA rate or at a
// weight-streaming rate this kernel does not beat.
//
// Why a kernel of its own: at M = 256 the four per-layer products carry 99 GFLOP
// over 386 MB of weights, so they sit at the ridge between the MFMA rate and HBM
// bandwidth, and their output (256 x N) is too small to give all 256 CUs a tile
// with enough operand reuse. hipBLASLt's choices reach 1.2-3 TB/s here.
//
// Design:
//   * one workgroup computes a BM x BN output tile over a K range (split-K when
//     the tiles alone cannot fill the chip; fp32 partials, then a reduce kernel);
//   * the x and w tiles of each 64-wide K step stream through a 3- to 5-deep LDS ring filled
//     by direct global -> LDS copies (global_load_lds_dwordx4), rows of 128 bytes
//     with the 16-byte chunks XOR-swizzled so the MFMA operand reads are
//     conflict-free;
//   * each wave owns a (32 a) x (32 b) block of the transposed product
//     D[n][m] = sum_k w[n][k] x[m][k] and runs v_mfma_f32_32x32x16 with A = w rows and
//     B = x rows, so each lane ends up with 4 consecutive output columns per
//     accumulator quad (8-byte stores);
//   * workgroups that share a weight tile (different M tiles of it) are placed on the
//     same XCD (workgroup i runs on XCD i mod 8), so the tile is fetched from HBM once.
#include <algorithm>
#include <mutex>
#include <cstdint>

#include "common.h"

namespace mi355x {
namespace {

typedef __bf16 lin_bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 lin_f16x8_t __attribute__((ext_vector_type(8)));
typedef float lin_floatx16 __attribute__((ext_vector_type(16)));

template <int DT>
__device__ __forceinline__ lin_floatx16 mfma32(const uint4& a, const uint4& b, lin_floatx16 c) {
  if constexpr (DT == 0)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(lin_bf16x8_t, a),
                                                   __builtin_bit_cast(lin_bf16x8_t, b), c, 0, 0,
                                                   0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(lin_f16x8_t, a),
                                                  __builtin_bit_cast(lin_f16x8_t, b), c, 0, 0, 0);
}

constexpr int kBK = 64;            // K elements per ring stage
constexpr int kRowBytes = kBK * 2;  // one tile row of a stage

struct LinearArgs {
  const uint16_t* x;
  const uint16_t* w;
  uint16_t* out;
  float* partial;  // [splits][M][N] fp32 when splits > 1
  int64_t ldx, ldw, ldo;
  int32_t M, N, K;
  int32_t splits, k_per_split;  // k_per_split is a multiple of kBK
  int32_t tiles_m, tiles_n, groups;  // groups = tiles_n * splits rounded up to 8
};

// Swizzled position of 16-byte chunk c in tile row r: c ^ f(r) with
// f(r) = (r & 7) ^ ((r >> 3) & 1). Any 8 consecutive rows (aligned) put a given chunk
// in 8 different positions, and over 16 rows the (row parity, position) pairs are all
// distinct, so 32 lanes reading one chunk of 32 rows hit every bank evenly.
__device__ __forceinline__ int chunk_pos(int c, int r) { return c ^ ((r & 7) ^ ((r >> 3) & 1)); }

// With SILU the product is a gate_up projection, w = [gate rows (N/2); up rows (N/2)], and
// the kernel writes silu(gate) * up ([M, N/2]) instead of the product: rows 8 q .. 8 q + 7 of
// each 32-row block of the weight tile come from gate for even q and from the matching up
// rows for odd q, so every lane holds gate column j and up column j side by side (see the
// epilogue) and the gate_up product never reaches memory.
__device__ __forceinline__ int silu_tile_row(int n0, int r, int half_n, bool* up) {
  const int rr = r & 31, q = rr >> 3;
  *up = (q & 1) != 0;
  return n0 / 2 + (r >> 5) * 16 + (q >> 1) * 8 + (rr & 7);  // output column
}

template <int DT, int BM, int BN, int WM, int WN, int STAGES, bool PARTIAL, bool SILU = false>
__global__ __launch_bounds__(64 * WM * WN, 1) void linear_kernel(LinearArgs a) {
  static_assert(!(SILU && PARTIAL), "the fused SiLU epilogue needs the whole K range");
  constexpr int NW = WM * WN;
  constexpr int kWaveM = BM / WM, kWaveN = BN / WN;  // wave tile
  constexpr int A_BLK = kWaveN / 32, B_BLK = kWaveM / 32;
  static_assert(kWaveM % 32 == 0 && kWaveN % 32 == 0, "wave tile must be 32-aligned");
  constexpr int kGroups = (BM + BN) / 8;  // 8-row (1 KB) copy groups per stage
  static_assert(kGroups % NW == 0, "copy groups must split evenly over the waves");
  constexpr int kCopies = kGroups / NW;  // copy instructions per wave per stage
  constexpr int kStageBytes = (BM + BN) * kRowBytes;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[STAGES * kStageBytes];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  if (a.M < 0) lds[tid] = 0;  // never taken; the copies' LDS writes are invisible

  // Workgroup -> (M tile, N tile, split). The M tiles of one (N tile, split) are
  // consecutive multiples of 8 apart, i.e. on one XCD at about the same time.
  const int b = blockIdx.x;
  const int xcd = b & 7;
  const int rest = b >> 3;
  const int tm = rest % a.tiles_m;
  const int lin = (rest / a.tiles_m) * 8 + xcd;
  if (lin >= a.tiles_n * a.splits) return;
  const int tn = lin % a.tiles_n;
  const int split = lin / a.tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  const int k_begin = split * a.k_per_split;
  const int n_k = min(a.k_per_split, a.K - k_begin) / kBK;

  const uint32_t lds_base = lds_address(lds);
  // Copy side: group g = wave + NW * j covers tile rows 8 g .. 8 g + 7 (x rows first,
  // then w rows); lane -> row 8 g + lane / 8, position lane % 8.
  const uint16_t* src[kCopies];
  uint32_t dst[kCopies];
#pragma unroll
  for (int j = 0; j < kCopies; ++j) {
    const int g = wave + NW * j;
    const int row = 8 * g + (lane >> 3);
    const int pos = lane & 7;
    if (8 * g < BM) {
      const int m = min(m0 + row, a.M - 1);
      src[j] = a.x + static_cast<int64_t>(m) * a.ldx + k_begin + chunk_pos(pos, row) * 8;
    } else {
      const int r = row - BM;
      int n;
      if constexpr (SILU) {
        bool up;
        const int oc = min(silu_tile_row(n0, r, a.N / 2, &up), a.N / 2 - 1);
        n = up ? a.N / 2 + oc : oc;
      } else {
        n = min(n0 + r, a.N - 1);
      }
      src[j] = a.w + static_cast<int64_t>(n) * a.ldw + k_begin + chunk_pos(pos, r) * 8;
    }
    dst[j] = lds_base + g * 1024;
  }
  auto issue = [&](int t, int stage) {
#pragma unroll
    for (int j = 0; j < kCopies; ++j) copy_to_lds(src[j] + t * kBK, dst[j] + stage * kStageBytes);
  };

  const int wm = wave % WM, wn = wave / WM;
  const int col = lane & 31, half = lane >> 5;
  lin_floatx16 acc[A_BLK][B_BLK];
#pragma unroll
  for (int i = 0; i < A_BLK; ++i)
#pragma unroll
    for (int j = 0; j < B_BLK; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // All operand fragments of a stage are read before its MFMAs (a scheduling barrier
  // keeps the compiler from interleaving them to save registers), so each MFMA waits
  // only for reads issued a whole k-step earlier rather than the one just before it.
  auto compute = [&](int stage) {
    const uint8_t* sb = lds + stage * kStageBytes;
    uint4 af[kBK / 16][A_BLK], bf[kBK / 16][B_BLK];
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      const int c = 2 * kk + half;
#pragma unroll
      for (int i = 0; i < A_BLK; ++i) {
        const int r = wn * kWaveN + 32 * i + col;
        af[kk][i] =
            *reinterpret_cast<const uint4*>(sb + (BM + r) * kRowBytes + chunk_pos(c, r) * 16);
      }
#pragma unroll
      for (int j = 0; j < B_BLK; ++j) {
        const int r = wm * kWaveM + 32 * j + col;
        bf[kk][j] = *reinterpret_cast<const uint4*>(sb + r * kRowBytes + chunk_pos(c, r) * 16);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk)
#pragma unroll
      for (int i = 0; i < A_BLK; ++i)
#pragma unroll
        for (int j = 0; j < B_BLK; ++j) acc[i][j] = mfma32<DT>(af[kk][i], bf[kk][j], acc[i][j]);
  };

#pragma unroll
  for (int st = 0; st < STAGES - 1; ++st)
    if (st < n_k) issue(st, st);
  int read_stage = 0, fill_stage = STAGES - 1;
  for (int t = 0; t < n_k; ++t) {
    wait_tiles_ahead<kCopies, STAGES - 2>(min(STAGES - 2, n_k - 1 - t));
    __syncthreads();
    if (t + STAGES - 1 < n_k) issue(t + STAGES - 1, fill_stage);
    compute(read_stage);
    read_stage = read_stage == STAGES - 1 ? 0 : read_stage + 1;
    fill_stage = fill_stage == STAGES - 1 ? 0 : fill_stage + 1;
  }

  // Lane holds D[n][m] for m = column `col` of each B block and n = 8 q + 4 half + e
  // (e = 0..3) of each A block, accumulator elements 4 q + e.
  if constexpr (SILU) {
    // Quads q (gate) and q + 1 (up) hold the same 4 output columns: round both as the
    // stand-alone product would, then silu(g) * u exactly as the stand-alone SiLU pass.
#pragma unroll
    for (int j = 0; j < B_BLK; ++j) {
      const int m = m0 + wm * kWaveM + 32 * j + col;
      if (m >= a.M) continue;
#pragma unroll
      for (int i = 0; i < A_BLK; ++i)
#pragma unroll
        for (int q = 0; q < 4; q += 2) {
          bool up;
          const int oc = silu_tile_row(n0, wn * kWaveN + 32 * i + 8 * q + 4 * half, a.N / 2, &up);
          if (oc >= a.N / 2) continue;
          float g[4], u[4], y[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            g[e] = Elem<DT>::to_float(Elem<DT>::from_float(acc[i][j][4 * q + e]));
            u[e] = Elem<DT>::to_float(Elem<DT>::from_float(acc[i][j][4 * q + 4 + e]));
            y[e] = (g[e] / (1.f + __expf(-g[e]))) * u[e];
          }
          const uint2 packed = make_uint2(Elem<DT>::pack2(y[0], y[1]), Elem<DT>::pack2(y[2], y[3]));
          *reinterpret_cast<uint2*>(a.out + static_cast<int64_t>(m) * a.ldo + oc) = packed;
        }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < B_BLK; ++j) {
    const int m = m0 + wm * kWaveM + 32 * j + col;
    if (m >= a.M) continue;
#pragma unroll
    for (int i = 0; i < A_BLK; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn * kWaveN + 32 * i + 8 * q + 4 * half;
        if (n >= a.N) continue;
        const float v[4] = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                            acc[i][j][4 * q + 3]};
        if constexpr (PARTIAL) {
          float* p = a.partial + (static_cast<int64_t>(split) * a.M + m) * a.N + n;
          *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
          const uint2 packed = make_uint2(Elem<DT>::pack2(v[0], v[1]), Elem<DT>::pack2(v[2], v[3]));
          *reinterpret_cast<uint2*>(a.out + static_cast<int64_t>(m) * a.ldo + n) = packed;
        }
      }
  }
}

// out[m][n..n+3] = sum over splits of partial[s][m][n..n+3], rounded once.
template <int DT>
__global__ __launch_bounds__(256) void linear_reduce(const float* __restrict__ partial,
                                                     uint16_t* __restrict__ out, int64_t ldo,
                                                     int M, int N, int splits) {
  const int64_t quads = static_cast<int64_t>(M) * (N / 4);
  const int64_t plane = static_cast<int64_t>(M) * N;
  for (int64_t i = blockIdx.x * int64_t(256) + threadIdx.x; i < quads;
       i += int64_t(gridDim.x) * 256) {
    const int m = static_cast<int>(i / (N / 4));
    const int n = static_cast<int>(i % (N / 4)) * 4;
    float4 s = *reinterpret_cast<const float4*>(partial + static_cast<int64_t>(m) * N + n);
    for (int k = 1; k < splits; ++k) {
      const float4 t =
          *reinterpret_cast<const float4*>(partial + k * plane + static_cast<int64_t>(m) * N + n);
      s.x += t.x;
      s.y += t.y;
      s.z += t.z;
      s.w += t.w;
    }
    *reinterpret_cast<uint2*>(out + static_cast<int64_t>(m) * ldo + n) =
        make_uint2(Elem<DT>::pack2(s.x, s.y), Elem<DT>::pack2(s.z, s.w));
  }
}

// Fused epilogue for a projection followed by the residual RMSNorm (o_proj and down of a
// decoder layer): y = round(sum of the split-K partials) (or y read back rounded when K is
// not split), residual <- round(y + residual), out <- round(rms(y + residual) * weight),
// the norm on the unrounded fp32 sum. One 256-lane workgroup per row, 8 columns per chunk,
// chunk c + 256 j per lane and the same two-level sum of squares as the stand-alone
// residual RMSNorm for these widths, so the results equal the two separate passes bit for
// bit.
// SPLITS > 0: that many K splits, all partial loads (and the residual and weight loads)
// issued before the first sum, so a row costs one memory round trip; 0: any count, read
// split after split.
template <int DT, int NCH, bool PARTIAL, int SPLITS>
__global__ __launch_bounds__(256) void reduce_add_rms(const float* __restrict__ partial,
                                                      int splits, uint16_t* out, int64_t ldo,
                                                      uint16_t* residual, int64_t ldr,
                                                      const uint16_t* __restrict__ weight,
                                                      int M, int N, float eps) {
  constexpr int kHeld = SPLITS > 0 ? SPLITS : 1;
  __shared__ float wave_ss[4];
  const int64_t row = blockIdx.x;
  const int chunks = N >> 3;
  const int64_t plane = static_cast<int64_t>(M) * N;
  float vals[NCH][8];
  uint4 wraw[NCH], rraw[NCH], oraw[NCH];
  float4 part[NCH][kHeld][2];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int chunk = threadIdx.x + c * 256;
    if (chunk >= chunks) continue;
    wraw[c] = ld128(weight + chunk * 8);
    if constexpr (PARTIAL) {
      const float* p = partial + row * N + chunk * 8;
#pragma unroll
      for (int k = 0; k < kHeld; ++k) {
        part[c][k][0] = *reinterpret_cast<const float4*>(p + k * plane);
        part[c][k][1] = *reinterpret_cast<const float4*>(p + k * plane + 4);
      }
    } else {
      oraw[c] = ld128(out + row * ldo + chunk * 8);
    }
    rraw[c] = ld128(residual + row * ldr + chunk * 8);
  }
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int chunk = threadIdx.x + c * 256;
    if (chunk >= chunks) continue;
    if constexpr (PARTIAL) {
      float4 lo = part[c][0][0], hi = part[c][0][1];
      auto add = [&](const float4& a, const float4& b) {
        lo.x += a.x;
        lo.y += a.y;
        lo.z += a.z;
        lo.w += a.w;
        hi.x += b.x;
        hi.y += b.y;
        hi.z += b.z;
        hi.w += b.w;
      };
      if constexpr (SPLITS > 0) {
#pragma unroll
        for (int k = 1; k < SPLITS; ++k) add(part[c][k][0], part[c][k][1]);
      } else {
        const float* p = partial + row * N + chunk * 8;
        for (int k = 1; k < splits; ++k)
          add(*reinterpret_cast<const float4*>(p + k * plane),
              *reinterpret_cast<const float4*>(p + k * plane + 4));
      }
      const float y[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      unpack8<DT>(pack8<DT>(y), vals[c]);  // the projection's output, rounded once
    } else {
      unpack8<DT>(oraw[c], vals[c]);
    }
    float r[8];
    unpack8<DT>(rraw[c], r);
#pragma unroll
    for (int i = 0; i < 8; ++i) vals[c][i] += r[i];
    st128(residual + row * ldr + chunk * 8, pack8<DT>(vals[c]));
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = fmaf(vals[c][i], vals[c][i], ss);
  }
  ss = wave_sum(ss);
  if (threadIdx.x % kWave == 0) wave_ss[threadIdx.x / kWave] = ss;
  __syncthreads();
  ss = (wave_ss[0] + wave_ss[1]) + (wave_ss[2] + wave_ss[3]);
  const float scale = rsqrtf(ss / static_cast<float>(N) + eps);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int chunk = threadIdx.x + c * 256;
    if (chunk < chunks) {
      float wf[8];
      unpack8<DT>(wraw[c], wf);
      float y[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = (vals[c][i] * scale) * wf[i];
      st128(out + row * ldo + chunk * 8, pack8<DT>(y));
    }
  }
}

template <int DT, int NCH, bool PARTIAL>
void launch_reduce_add_rms_splits(const float* partial, int splits, uint16_t* out, int64_t ldo,
                                  uint16_t* residual, int64_t ldr, const uint16_t* weight,
                                  int M, int N, float eps, hipStream_t s) {
  const dim3 grid(static_cast<uint32_t>(M)), block(256);
#define MI355X_REDUCE_ADD_RMS(S)                                                            \
  reduce_add_rms<DT, NCH, PARTIAL, S><<<grid, block, 0, s>>>(partial, splits, out, ldo,    \
                                                             residual, ldr, weight, M, N, eps)
  if (!PARTIAL || splits == 1)
    MI355X_REDUCE_ADD_RMS(1);
  else if (splits == 2)
    MI355X_REDUCE_ADD_RMS(2);
  else if (splits == 4)
    MI355X_REDUCE_ADD_RMS(4);
  else
    MI355X_REDUCE_ADD_RMS(0);
#undef MI355X_REDUCE_ADD_RMS
}

template <int DT, bool PARTIAL>
void launch_reduce_add_rms(const float* partial, int splits, uint16_t* out, int64_t ldo,
                           uint16_t* residual, int64_t ldr, const uint16_t* weight, int M, int N,
                           float eps, hipStream_t s) {
  const int chunks = N / 8;
  if (chunks <= 256)
    launch_reduce_add_rms_splits<DT, 1, PARTIAL>(partial, splits, out, ldo, residual, ldr,
                                                 weight, M, N, eps, s);
  else if (chunks <= 512)
    launch_reduce_add_rms_splits<DT, 2, PARTIAL>(partial, splits, out, ldo, residual, ldr,
                                                 weight, M, N, eps, s);
  else
    launch_reduce_add_rms_splits<DT, 4, PARTIAL>(partial, splits, out, ldo, residual, ldr,
                                                 weight, M, N, eps, s);
}

struct TileConfig {
  int bm, bn, wm, wn, stages;
};

// The compiled tile shapes (waves arranged wm x wn over the tile).
constexpr TileConfig kConfigs[] = {
    {128, 192, 4, 2, 4},  // wave 32 x 96
    {128, 128, 4, 2, 5},  // wave 32 x 64
    {256, 128, 4, 2, 3},  // wave 64 x 64
    {128, 256, 4, 2, 3},  // wave 32 x 128
    {64, 256, 2, 4, 4},   // wave 32 x 64
    {256, 64, 8, 1, 4},   // wave 32 x 64
    {128, 128, 4, 2, 3},  // wave 32 x 64, shallow ring
    {64, 128, 2, 4, 5},   // wave 32 x 32
};
constexpr int kNumConfigs = sizeof(kConfigs) / sizeof(kConfigs[0]);

template <int DT, int C, bool PARTIAL>
void launch_config(const LinearArgs& a, int blocks, hipStream_t s) {
  constexpr TileConfig t = kConfigs[C];
  linear_kernel<DT, t.bm, t.bn, t.wm, t.wn, t.stages, PARTIAL>
      <<<dim3(blocks), dim3(64 * t.wm * t.wn), 0, s>>>(a);
}

template <int DT, int C>
void launch_any(const LinearArgs& a, int blocks, hipStream_t s) {
  if (a.splits > 1)
    launch_config<DT, C, true>(a, blocks, s);
  else
    launch_config<DT, C, false>(a, blocks, s);
}

template <int DT>
void launch_dt(int config, const LinearArgs& a, int blocks, hipStream_t s) {
  switch (config) {
    case 0: launch_any<DT, 0>(a, blocks, s); break;
    case 1: launch_any<DT, 1>(a, blocks, s); break;
    case 2: launch_any<DT, 2>(a, blocks, s); break;
    case 3: launch_any<DT, 3>(a, blocks, s); break;
    case 4: launch_any<DT, 4>(a, blocks, s); break;
    case 5: launch_any<DT, 5>(a, blocks, s); break;
    case 6: launch_any<DT, 6>(a, blocks, s); break;
    default: launch_any<DT, 7>(a, blocks, s); break;
  }
}

// The fused gate_up + SiLU launches (never split: K whole in every workgroup), for the
// tile shapes `choose` can pick.
template <int DT>
bool launch_silu(int config, const LinearArgs& a, int blocks, hipStream_t s) {
  switch (config) {
    case 0:
      linear_kernel<DT, 128, 192, 4, 2, 4, false, true><<<dim3(blocks), dim3(512), 0, s>>>(a);
      return true;
    case 6:
      linear_kernel<DT, 128, 128, 4, 2, 3, false, true><<<dim3(blocks), dim3(512), 0, s>>>(a);
      return true;
    case 7:
      linear_kernel<DT, 64, 128, 2, 4, 5, false, true><<<dim3(blocks), dim3(512), 0, s>>>(a);
      return true;
    default:
      return false;
  }
}

struct Choice {
  int config, splits;
};

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Tile shape and split count: for each tile shape in order of preference, the fewest
// K splits that give at least 3/4 of a workgroup per CU; the first shape that needs at
// most 4 splits wins, else the one needing the fewest. Measured on MI355X at the
// Qwen3-8B decode shapes (M = 1..256) with the weights streamed from HBM (rotating over
// more than 1 GB): 128 x 128 tiles with up to 4 splits beat smaller tiles with fewer
// splits at 128-192 rows (QKV at 192 rows 27.7 us against 29.8 for 64 x 128 tiles
// unsplit) and tie with them at 256 rows; the long-K down projection gains most.
Choice choose(int64_t M, int64_t N, int64_t K, int cus) {
  const int order[] = {6, 0, 7};
  const int64_t want = (3 * int64_t(cus)) / 4;
  Choice best{-1, 1 << 30};
  for (int c : order) {
    const TileConfig& t = kConfigs[c];
    const int64_t tiles = ceil_div(M, t.bm) * ceil_div(N, t.bn);
    int s = 1;
    while (s < 8 && tiles * s < want && K % (int64_t(2 * s) * kBK) == 0) s *= 2;
    if (K % (int64_t(s) * kBK)) continue;
    if (s <= 4) return {c, s};
    if (s < best.splits) best = {c, s};
  }
  return best.config >= 0 ? best : Choice{7, 1};
}

}  // namespace
}  // namespace mi355x

using namespace mi355x;

// Workspace bytes (fp32 split-K partials) that mi355x_linear needs for this shape.
extern "C" int64_t mi355x_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t cus,
                                                 int32_t config, int32_t splits) {
  if (M <= 0 || N <= 0 || K <= 0) return -1;
  Choice c = config >= 0 ? Choice{config, splits} : choose(M, N, K, cus > 0 ? cus : 256);
  return c.splits > 1 ? int64_t(c.splits) * M * N * 4 : 0;
}

namespace mi355x {
// Validates, picks the tiling and launches the projection. With `leave_partials` the
// split-K partials are left in the workspace (no reduce) and `*splits_used` tells how many
// (1: the product went straight to `out`). Shared with the fused QKV pass in layer_ops.hip.
const char* run_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, void* out,
                       int64_t ldo, int64_t M, int64_t N, int64_t K, void* workspace,
                       int64_t workspace_bytes, int32_t cus, int32_t config, int32_t splits,
                       int64_t dtype, bool leave_partials, int* splits_used, hipStream_t s) {
  if (!x || !w || !out) return set_error("mi355x_linear: null pointer");
  if (M <= 0 || N <= 0 || K <= 0 || M > 4096 || N % 4 || K % kBK || ldx < K || ldw < K ||
      ldo < N || ldx % 8 || ldw % 8 || ldo % 4 || (dtype != 0 && dtype != 1))
    return set_error("mi355x_linear: unsupported shape (K % 64, N % 4, 16-byte rows)");
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(out, 8))
    return set_error("mi355x_linear: misaligned operand");
  Choice c = config >= 0 ? Choice{config, splits} : choose(M, N, K, cus > 0 ? cus : 256);
  if (c.config < 0 || c.config >= kNumConfigs || c.splits < 1 || K % (int64_t(c.splits) * kBK))
    return set_error("mi355x_linear: invalid tile configuration");
  const TileConfig& t = kConfigs[c.config];
  if (c.splits > 1) {
    if (!workspace || workspace_bytes < int64_t(c.splits) * M * N * 4 || !aligned(workspace, 16))
      return set_error("mi355x_linear: split-K workspace too small");
  }
  LinearArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(w);
  a.out = static_cast<uint16_t*>(out);
  a.partial = static_cast<float*>(workspace);
  a.ldx = ldx;
  a.ldw = ldw;
  a.ldo = ldo;
  a.M = static_cast<int32_t>(M);
  a.N = static_cast<int32_t>(N);
  a.K = static_cast<int32_t>(K);
  a.splits = c.splits;
  a.k_per_split = static_cast<int32_t>(K / c.splits);
  a.tiles_m = static_cast<int32_t>(ceil_div(M, t.bm));
  a.tiles_n = static_cast<int32_t>(ceil_div(N, t.bn));
  a.groups = static_cast<int32_t>(ceil_div(int64_t(a.tiles_n) * a.splits, 8) * 8);
  const int64_t blocks = int64_t(a.groups) * a.tiles_m;
  if (blocks > (int64_t(1) << 31) - 1) return set_error("mi355x_linear: grid too large");
  if (dtype == 0)
    launch_dt<0>(c.config, a, static_cast<int>(blocks), s);
  else
    launch_dt<1>(c.config, a, static_cast<int>(blocks), s);
  if (const char* e = launch_status("linear_kernel")) return e;
  if (splits_used) *splits_used = c.splits;
  if (c.splits > 1 && !leave_partials) {
    const int64_t quads = M * (N / 4);
    const int grid = static_cast<int>(std::min<int64_t>(ceil_div(quads, 256), 4096));
    if (dtype == 0)
      linear_reduce<0><<<grid, 256, 0, s>>>(a.partial, a.out, ldo, a.M, a.N, c.splits);
    else
      linear_reduce<1><<<grid, 256, 0, s>>>(a.partial, a.out, ldo, a.M, a.N, c.splits);
    if (const char* e = launch_status("linear_reduce")) return e;
  }
  return nullptr;
}
}  // namespace mi355x

extern "C" const char* mi355x_linear(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                     void* out, int64_t ldo, int64_t M, int64_t N, int64_t K,
                                     void* workspace, int64_t workspace_bytes, int32_t cus,
                                     int32_t config, int32_t splits, int64_t dtype,
                                     void* stream) {
  return run_linear(x, ldx, w, ldw, out, ldo, M, N, K, workspace, workspace_bytes, cus, config,
                    splits, dtype, false, nullptr, static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// Allocation-free variant of mi355x_linear: the split-K partials go to a file-scope
// device array instead of a caller workspace. Each GPU the library runs on holds its
// own copy of the array (kLinearScratchBytes) until the process ends. In host code the
// array's name is only a stand-in for its symbol; the device address of each GPU's copy
// is looked up once per device (hipGetSymbolAddress, with that device current) and that
// pointer is what the kernels receive.
// ---------------------------------------------------------------------------
namespace mi355x {
namespace {
constexpr int64_t kLinearScratchBytes = int64_t(32) << 20;
static __device__ __align__(256) uint8_t scratch[kLinearScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch array, looked up on first use.
const char* scratch_for_current_device(void** out) {
  int device = 0;
  hipError_t st = hipGetDevice(&device);
  if (st != hipSuccess) return hip_error(st, "hipGetDevice");
  if (device < 0 || device >= kMaxDevices) return set_error("mi355x_linear_noalloc: device id");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[device]) {
    void* ptr = nullptr;
    st = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (st != hipSuccess) return hip_error(st, "hipGetSymbolAddress(scratch)");
    g_scratch_ptr[device] = ptr;
  }
  *out = g_scratch_ptr[device];
  return nullptr;
}
}  // namespace
}  // namespace mi355x

extern "C" const char* mi355x_linear_noalloc(const void* x, int64_t ldx, const void* w,
                                             int64_t ldw, void* out, int64_t ldo, int64_t M,
                                             int64_t N, int64_t K, int32_t cus, int32_t config,
                                             int32_t splits, int64_t dtype, void* stream) {
  const int64_t need = mi355x_linear_workspace_bytes(M, N, K, cus, config, splits);
  if (need < 0) return set_error("mi355x_linear: unsupported shape (K % 64, N % 4, 16-byte rows)");
  if (need > kLinearScratchBytes)
    return set_error("mi355x_linear_noalloc: split-K partials exceed the 32 MiB scratch "
                     "(use mi355x_linear with a workspace)");
  void* ws = nullptr;
  if (need > 0) {
    if (const char* e = scratch_for_current_device(&ws)) return e;
  }
  // Every split writes its whole [M, N] slice of partials before the reduce reads it,
  // so the scratch needs no clearing between calls.
  return run_linear(x, ldx, w, ldw, out, ldo, M, N, K, ws, need, cus, config, splits, dtype,
                    false, nullptr, static_cast<hipStream_t>(stream));
}

extern "C" const char* mi355x_linear_add_rms_norm(const void* x, int64_t ldx, const void* w,
                                                  int64_t ldw, void* residual, int64_t ldr,
                                                  const void* norm_weight, double eps, void* out,
                                                  int64_t ldo, int64_t M, int64_t N, int64_t K,
                                                  void* workspace, int64_t workspace_bytes,
                                                  int32_t cus, int64_t dtype, void* stream) {
  if (!residual || !norm_weight) return set_error("mi355x_linear_add_rms_norm: null pointer");
  if (N % 8 || N / 8 <= 128 || N / 8 > 1024 || ldr < N || ldr % 8 || ldo % 8 ||
      !aligned(residual, 16) || !aligned(out, 16) || !aligned(norm_weight, 16))
    return set_error("mi355x_linear_add_rms_norm: width must be 1032..8192 in 16-byte rows");
  if (out == residual)  // the norm pass reads and writes both
    return set_error("mi355x_linear_add_rms_norm: out and residual must not alias");
  auto s = static_cast<hipStream_t>(stream);
  int used = 1;
  if (const char* e = run_linear(x, ldx, w, ldw, out, ldo, M, N, K, workspace, workspace_bytes,
                                 cus, -1, -1, dtype, true, &used, s))
    return e;
  const float* partial = static_cast<const float*>(workspace);
  auto* o = static_cast<uint16_t*>(out);
  auto* r = static_cast<uint16_t*>(residual);
  const auto* g = static_cast<const uint16_t*>(norm_weight);
  const int m = static_cast<int>(M), n = static_cast<int>(N);
  const float fe = static_cast<float>(eps);
  if (dtype == 0) {
    if (used > 1)
      launch_reduce_add_rms<0, true>(partial, used, o, ldo, r, ldr, g, m, n, fe, s);
    else
      launch_reduce_add_rms<0, false>(partial, 1, o, ldo, r, ldr, g, m, n, fe, s);
  } else {
    if (used > 1)
      launch_reduce_add_rms<1, true>(partial, used, o, ldo, r, ldr, g, m, n, fe, s);
    else
      launch_reduce_add_rms<1, false>(partial, 1, o, ldo, r, ldr, g, m, n, fe, s);
  }
  return launch_status("reduce_add_rms");
}

extern "C" const char* mi355x_linear_silu_mul(const void* x, int64_t ldx, const void* w,
                                              int64_t ldw, void* out, int64_t ldo, int64_t M,
                                              int64_t width, int64_t K, int32_t cus,
                                              int32_t config, int64_t dtype, void* stream) {
  if (!x || !w || !out) return set_error("mi355x_linear_silu_mul: null pointer");
  const int64_t N = 2 * width;
  if (M <= 0 || width <= 0 || M > 4096 || width % 4 || K <= 0 || K % kBK || ldx < K ||
      ldw < K || ldo < width || ldx % 8 || ldw % 8 || ldo % 4 || N > (int64_t(1) << 30) ||
      (dtype != 0 && dtype != 1))
    return set_error("mi355x_linear_silu_mul: unsupported shape (K % 64, width % 4, 16-byte rows)");
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(out, 8))
    return set_error("mi355x_linear_silu_mul: misaligned operand");
  // Tile shape measured on MI355X at the Qwen3-8B gate_up shape (width 12288, K 4096):
  // 128 x 192 tiles from 129 rows up (62.6 us at 256 rows against 66.5 for hipBLASLt plus
  // the SiLU pass), 128 x 128 for 65..128 rows, 64 x 128 below.
  if (config < 0) config = M > 128 ? 0 : (M > 64 ? 6 : 7);
  if (config >= kNumConfigs) return set_error("mi355x_linear_silu_mul: invalid tile configuration");
  const TileConfig& t = kConfigs[config];
  LinearArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(w);
  a.out = static_cast<uint16_t*>(out);
  a.ldx = ldx;
  a.ldw = ldw;
  a.ldo = ldo;
  a.M = static_cast<int32_t>(M);
  a.N = static_cast<int32_t>(N);
  a.K = static_cast<int32_t>(K);
  a.splits = 1;
  a.k_per_split = static_cast<int32_t>(K);
  a.tiles_m = static_cast<int32_t>(ceil_div(M, t.bm));
  a.tiles_n = static_cast<int32_t>(ceil_div(N, t.bn));
  a.groups = static_cast<int32_t>(ceil_div(a.tiles_n, 8) * 8);
  const int64_t blocks = int64_t(a.groups) * a.tiles_m;
  if (blocks > (int64_t(1) << 31) - 1) return set_error("mi355x_linear_silu_mul: grid too large");
  auto s = static_cast<hipStream_t>(stream);
  const bool ok = dtype == 0 ? launch_silu<0>(config, a, static_cast<int>(blocks), s)
                             : launch_silu<1>(config, a, static_cast<int>(blocks), s);
  if (!ok) return set_error("mi355x_linear_silu_mul: no fused kernel for this tiling");
  return launch_status("linear_kernel (silu)");
}
