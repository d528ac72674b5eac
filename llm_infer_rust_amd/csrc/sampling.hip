// Joint top-k / top-p token sampling for gfx950, one workgroup per logits row.
//
// Semantics (src/engine/sampling.rs:239-269, 330-372, 409-428):
//   * parameters are normalised as SamplingParams::normalized does: a top_p
//     that is not finite or lies outside [0, 1] becomes 1; top_k <= 0 or
//     top_k > vocab means the whole vocabulary;
//   * temperature <= 0 or top_p == 0 -> argmax of the raw logits (first index
//     of the maximum, NaN counting as the maximum, as torch's argmax);
//   * otherwise s = cast(logit * (1 / temperature)) in the logits dtype (a
//     tensor divided by a scalar is computed as a multiply by the fp32
//     reciprocal on the GPU) and p = softmax(s) in fp32; both cutoffs are taken on that ORIGINAL p:
//       top-k keeps p >= (k-th largest p)       (ties at the boundary kept)
//       top-p keeps p >= v*, v* = the largest value whose "mass at or above"
//             reaches top_p; when rounding keeps every prefix below top_p the
//             smallest p is the cutoff (the reference's clamp to vocab-1);
//     a token survives when it passes both, and one token is drawn from the
//     surviving p renormalised;
//   * a row whose distribution is invalid (NaN anywhere, every logit -inf, or a scaled
//     logit of +inf, which makes the reference's softmax NaN) yields -1, the
//     reference's invalid-distribution sentinel
//     (sampling_bridge.cpp: output.masked_fill_(!valid, -1)).
//
// Algorithm:
//   pass 1  row max and sum of exp (online), NaN detection;
//   pass 2-4 radix selection over the fp32 bit pattern of p (non-negative, so
//     the bits order like the values), 12 + 10 + 9 bits. Each pass builds a
//     count histogram (top-k) and a mass histogram (top-p) in LDS and a
//     workgroup suffix scan picks the bin holding the cutoff. Mass is summed in
//     64-bit fixed point (2^-40 units) so the histogram, and hence the cutoff,
//     does not depend on the order of the LDS atomics: equal seeds give equal
//     tokens;
//   pass 5  exponential race: the surviving token with the largest s + G,
//     G = -log(-log(u)) a Gumbel variate, is an exact draw from the surviving
//     distribution (Gumbel-max). u comes from Philox4x32-10 (Salmon et al.,
//     SC'11) keyed by the seed, with counter (element/4, row, offset), so the
//     draw needs no prefix scan and no renormalising sum.
// Without either cutoff only the race pass runs; greedy rows run one argmax pass.
#include "common.h"

namespace mi355x {
namespace {

constexpr int kThreads = 1024;
constexpr int kWarps = kThreads / kWave;
constexpr int kBins0 = 4096;  // bits 30..19 of p (bit 31, the sign, is always 0)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kFixedScale = 1099511627776.0f;  // 2^40
constexpr uint32_t kCandidates = 2048;  // candidate path: (index, s, p) lists in LDS

// Logits element access for dtype codes 0 (bf16), 1 (fp16), 2 (fp32).
template <int DT>
struct Logit {
  using Word = uint16_t;
  static constexpr int kVec = 8;
  __device__ __forceinline__ static float to_float(Word w) { return Elem<DT>::to_float(w); }
  __device__ __forceinline__ static float round(float f) {
    return Elem<DT>::to_float(Elem<DT>::from_float(f));
  }
};
template <>
struct Logit<2> {
  using Word = float;
  static constexpr int kVec = 4;
  __device__ __forceinline__ static float to_float(Word w) { return w; }
  // The scaled logit must be the rounded product: without the barrier the compiler may fuse
  // x * (1 / T) into a later s - max as one fma, which differs from the rounded s by up to half
  // an ulp, and can differ between the passes (the top token's p then missing its own cutoff).
  __device__ __forceinline__ static float round(float f) {
    asm volatile("" : "+v"(f));
    return f;
  }
};

// Philox4x32-10 (Random123): 10 rounds, key schedule bumped between rounds.
__device__ __forceinline__ uint4 philox4x32_10(uint4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r > 0) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint32_t lo0 = 0xD2511F53u * c.x, hi0 = __umulhi(0xD2511F53u, c.x);
    const uint32_t lo1 = 0xCD9E8D57u * c.z, hi1 = __umulhi(0xCD9E8D57u, c.z);
    c = make_uint4(hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0);
  }
  return c;
}

// Uniform in (0, 1) from 23 random bits, then a Gumbel variate.
__device__ __forceinline__ float gumbel(uint32_t bits) {
  const float u = (static_cast<float>(bits >> 9) + 0.5f) * 1.1920928955078125e-07f;  // 2^-23
  return -__logf(-__logf(u));
}

struct SampleArgs {
  const void* logits;
  int64_t rows, vocab, stride;
  const float* temperature;
  const int32_t* top_k;
  const float* top_p;
  uint32_t seed_lo, seed_hi, offset_lo, offset_hi;
  int64_t* out;
};

// Workgroup reductions through a small LDS scratch array.
struct Shared {
  uint32_t cnt[kBins0];
  unsigned long long mass[kBins0];
  float red_f[kWarps];
  float red_g[kWarps];
  int64_t red_i[kWarps];
  uint32_t scan_c[kWarps];
  unsigned long long scan_m[kWarps];
  // Selection state broadcast to the workgroup.
  uint32_t k_prefix, k_rem, p_prefix, p_lowest;
  unsigned long long p_rem;
  int p_found, k_found, k_active;
};

// Unsigned key that orders like the float value (non-NaN): larger s, larger key.
__device__ __forceinline__ uint32_t order_key(float s) {
  const uint32_t u = __float_as_uint(s);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t key) {
  return __uint_as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

__device__ __forceinline__ bool better(float v, int64_t i, float bv, int64_t bi) {
  // Larger value wins, NaN beats everything, lower index breaks ties.
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

__device__ void block_argmax(Shared& sh, float& v, int64_t& i) {
  const int lane = threadIdx.x % kWave, warp = threadIdx.x / kWave;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(v, off);
    const int64_t oi = __shfl_xor(i, off);
    if (better(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
  if (lane == 0) {
    sh.red_f[warp] = v;
    sh.red_i[warp] = i;
  }
  __syncthreads();
  v = sh.red_f[0];
  i = sh.red_i[0];
  for (int w = 1; w < kWarps; ++w)
    if (better(sh.red_f[w], sh.red_i[w], v, i)) {
      v = sh.red_f[w];
      i = sh.red_i[w];
    }
  __syncthreads();
}

// Visit every element of the row as (index, value). The vector body uses
// 128-bit loads when the row is aligned; a scalar loop covers the rest.
template <int DT, typename F>
__device__ __forceinline__ void for_each(const SampleArgs& a, int64_t row, bool vec, F&& f) {
  using L = Logit<DT>;
  using W = typename L::Word;
  const W* base = static_cast<const W*>(a.logits) + row * a.stride;
  int64_t start = 0;
  if (vec) {
    const int64_t groups = a.vocab / L::kVec;
    for (int64_t g = threadIdx.x; g < groups; g += kThreads) {
      const uint4 raw = ld128(base + g * L::kVec);
      const W* w = reinterpret_cast<const W*>(&raw);
#pragma unroll
      for (int j = 0; j < L::kVec; ++j) f(g * L::kVec + j, L::to_float(w[j]));
    }
    start = groups * L::kVec;
  }
  for (int64_t i = start + threadIdx.x; i < a.vocab; i += kThreads) f(i, L::to_float(base[i]));
}

// Inclusive workgroup prefix sum of (count, mass) in thread order.
__device__ void block_scan(Shared& sh, uint32_t& c, unsigned long long& m, uint32_t& total_c,
                           unsigned long long& total_m) {
  const int lane = threadIdx.x % kWave, warp = threadIdx.x / kWave;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const uint32_t oc = __shfl_up(c, off);
    const unsigned long long om = __shfl_up(m, off);
    if (lane >= off) {
      c += oc;
      m += om;
    }
  }
  if (lane == kWave - 1) {
    sh.scan_c[warp] = c;
    sh.scan_m[warp] = m;
  }
  __syncthreads();
  uint32_t pc = 0;
  unsigned long long pm = 0;
  total_c = 0;
  total_m = 0;
  for (int w = 0; w < kWarps; ++w) {
    if (w < warp) {
      pc += sh.scan_c[w];
      pm += sh.scan_m[w];
    }
    total_c += sh.scan_c[w];
    total_m += sh.scan_m[w];
  }
  c += pc;
  m += pm;
  __syncthreads();
}

template <int DT>
__global__ __launch_bounds__(kThreads) void sample_kernel(SampleArgs a, bool vec) {
  __shared__ Shared sh;
  const int64_t row = blockIdx.x;
  const int64_t vocab = a.vocab;

  float temperature = a.temperature[row];
  float top_p = a.top_p[row];
  if (!(top_p >= 0.f && top_p <= 1.f)) top_p = 1.f;  // NaN/inf/out of range -> 1
  int64_t top_k = a.top_k[row];
  if (top_k <= 0 || top_k > vocab) top_k = vocab;

  if (temperature <= 0.f || top_p == 0.f) {
    float bv = -INFINITY;
    int64_t bi = vocab;  // any real index beats the sentinel
    bool first = true;
    for_each<DT>(a, row, vec, [&](int64_t i, float x) {
      if (first || better(x, i, bv, bi)) {
        bv = x;
        bi = i;
        first = false;
      }
    });
    block_argmax(sh, bv, bi);
    if (threadIdx.x == 0) a.out[row] = bi < vocab ? bi : 0;
    return;
  }

  using L = Logit<DT>;
  const float inv_t = 1.f / temperature;
  auto scaled = [&](float x) { return L::round(x * inv_t); };
  const bool filter = top_k < vocab || top_p < 1.f;
  const uint32_t k0 = a.seed_lo, k1 = a.seed_hi;

  // Race over the survivors of `keep`; also reports whether a NaN was seen.
  auto race = [&](auto keep, bool& nan_seen, float& best, int64_t& best_i) {
    best = -INFINITY;
    best_i = vocab;
    int64_t cached_group = -1;
    uint4 rnd = make_uint4(0, 0, 0, 0);
    for_each<DT>(a, row, vec, [&](int64_t i, float x) {
      const float s = scaled(x);
      if (s != s || s == INFINITY) nan_seen = true;
      if (!keep(s) || s == -INFINITY) return;
      const int64_t group = i >> 2;
      if (group != cached_group) {
        rnd = philox4x32_10(make_uint4(static_cast<uint32_t>(group), static_cast<uint32_t>(row),
                                       a.offset_lo, a.offset_hi),
                            k0, k1);
        cached_group = group;
      }
      const uint32_t words[4] = {rnd.x, rnd.y, rnd.z, rnd.w};
      const float key = s + gumbel(words[i & 3]);
      if (key > best || (key == best && i < best_i)) {
        best = key;
        best_i = i;
      }
    });
  };

  if (!filter) {
    bool nan_seen = false;
    float best;
    int64_t best_i;
    race([](float) { return true; }, nan_seen, best, best_i);
    const int any_nan = __syncthreads_or(nan_seen);
    block_argmax(sh, best, best_i);
    if (threadIdx.x == 0) a.out[row] = (any_nan || best_i >= vocab) ? -1 : best_i;
    return;
  }

  // Top-k rows first try a shorter route (the candidate path below); pass 1 then also
  // counts the scaled logits in 4,096 bins of their top order-key bits.
  const bool fast_k = top_k < vocab;
  if (fast_k) {
    for (int b = threadIdx.x; b < kBins0; b += kThreads) sh.cnt[b] = 0;
    __syncthreads();
  }
  // Pass 1: max and sum of exp(s - max).
  float m = -INFINITY, z = 0.f;
  bool nan_seen = false;
  for_each<DT>(a, row, vec, [&](int64_t, float x) {
    const float s = scaled(x);
    if (fast_k && s == s && s != -INFINITY) atomicAdd(&sh.cnt[order_key(s) >> 20], 1u);
    if (s != s || s == INFINITY) {  // softmax of a row holding +inf is NaN throughout
      nan_seen = true;
      return;
    }
    if (s == -INFINITY) return;
    if (s > m) {
      z = z * exp2f((m - s) * kLog2e) + 1.f;
      m = s;
    } else {
      z += exp2f((s - m) * kLog2e);
    }
  });
  {
    const int lane = threadIdx.x % kWave, warp = threadIdx.x / kWave;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float om = __shfl_xor(m, off), oz = __shfl_xor(z, off);
      const float nm = fmaxf(m, om);
      z = (m == -INFINITY ? 0.f : z * exp2f((m - nm) * kLog2e)) +
          (om == -INFINITY ? 0.f : oz * exp2f((om - nm) * kLog2e));
      m = nm;
    }
    if (lane == 0) {
      sh.red_f[warp] = m;
      sh.red_g[warp] = z;
    }
    const int any_nan = __syncthreads_or(nan_seen);
    m = -INFINITY;
    for (int w = 0; w < kWarps; ++w) m = fmaxf(m, sh.red_f[w]);
    z = 0.f;
    for (int w = 0; w < kWarps; ++w)
      if (sh.red_f[w] != -INFINITY) z += sh.red_g[w] * exp2f((sh.red_f[w] - m) * kLog2e);
    __syncthreads();
    if (any_nan || m == -INFINITY || !(z > 0.f)) {
      if (threadIdx.x == 0) a.out[row] = -1;
      return;
    }
  }
  const float inv_z = 1.f / z;
  auto prob = [&](float s) { return exp2f((s - m) * kLog2e) * inv_z; };
  auto fixed = [](float p) { return static_cast<unsigned long long>(p * kFixedScale + 0.5f); };
  const bool use_p = top_p < 1.f;
  const unsigned long long p_target = [&] {
    const unsigned long long t = static_cast<unsigned long long>(top_p * kFixedScale);
    return t ? t : 1ull;  // at least one unit, so the top bin is always selectable
  }();

  // Candidate path (top-k rows): the order-key histogram of pass 1 gives the bin b1 that
  // holds the k-th largest scaled logit. Every token with s >= s_lo (the bin's lower edge
  // less a margin far above the rounding of p) is a candidate, and every other token's p is
  // below every candidate's that lies in or above b1, so the k-th largest p of the row, the
  // top-p cutoff at or above it (its mass in the same 2^-40 fixed point) and the survivors
  // are all found among the candidates, which are gathered once into LDS. Exactly the
  // cutoffs and draw of the radix path below; that path runs when the candidates do not
  // fit (heavy ties), a row has fewer than k finite logits, or the k-th p has no fixed-point
  // mass. Two row passes instead of four, one of them without exponentials.
  if (fast_k) {
    // Bin b1 from the top, through the same thread-owns-4-bins suffix scan as below.
    const int b0 = threadIdx.x * 4;
    uint32_t c4[4];
    for (int j = 0; j < 4; ++j) c4[j] = sh.cnt[b0 + j];
    uint32_t csum = c4[0] + c4[1] + c4[2] + c4[3];
    unsigned long long zero = 0;
    uint32_t total_c;
    unsigned long long total_m;
    block_scan(sh, csum, zero, total_c, total_m);
    uint32_t c_above = total_c - csum;
    if (threadIdx.x == 0) sh.k_found = 0;
    __syncthreads();
    for (int j = 3; j >= 0; --j) {
      if (c4[j] && c_above < static_cast<uint32_t>(top_k) &&
          c_above + c4[j] >= static_cast<uint32_t>(top_k)) {
        sh.k_prefix = static_cast<uint32_t>(b0 + j);
        sh.k_rem = c_above + c4[j];  // tokens in bins b1 and above
        sh.k_found = 1;
      }
      c_above += c4[j];
    }
    __syncthreads();
    bool ok = sh.k_found && sh.k_rem <= kCandidates;
    if (ok) {
      const float s_lower = key_value(sh.k_prefix << 20);
      const float s_lo = s_lower - (fabsf(s_lower - m) + 1.f) * 0x1p-12f;
      uint32_t* cand_i = reinterpret_cast<uint32_t*>(sh.mass);
      float* cand_s = reinterpret_cast<float*>(cand_i + kCandidates);
      float* cand_p = cand_s + kCandidates;
      if (threadIdx.x == 0) sh.p_lowest = 0;  // candidate count
      __syncthreads();
      for_each<DT>(a, row, vec, [&](int64_t i, float x) {
        const float s = scaled(x);
        if (!(s >= s_lo) || s == -INFINITY) return;
        const uint32_t slot = atomicAdd(&sh.p_lowest, 1u);
        if (slot < kCandidates) {
          cand_i[slot] = static_cast<uint32_t>(i);
          cand_s[slot] = s;
        }
      });
      __syncthreads();
      const uint32_t n = sh.p_lowest;
      ok = n <= kCandidates;
      if (ok) {
        for (uint32_t t = threadIdx.x; t < n; t += kThreads) cand_p[t] = prob(cand_s[t]);
        __syncthreads();
        // The k-th largest p: the candidate value v with #(p > v) < k <= #(p >= v).
        if (threadIdx.x == 0) sh.k_found = 0;
        __syncthreads();
        for (uint32_t t = threadIdx.x; t < n; t += kThreads) {
          const float v = cand_p[t];
          uint32_t gt = 0, ge = 0;
          for (uint32_t u = 0; u < n; ++u) {
            gt += cand_p[u] > v;
            ge += cand_p[u] >= v;
          }
          if (gt < static_cast<uint32_t>(top_k) && ge >= static_cast<uint32_t>(top_k)) {
            sh.red_f[0] = v;  // every thread that gets here writes the same value
            sh.k_found = 1;
          }
        }
        __syncthreads();
        const float p_k = sh.red_f[0];
        ok = sh.k_found && !(use_p && fixed(p_k) == 0);
        float cut = p_k;
        if (ok && use_p) {
          // Mass at or above p_k; when it reaches top_p, the top-p cutoff is the largest
          // candidate value whose mass at or above reaches it.
          unsigned long long mk = 0;
          for (uint32_t t = threadIdx.x; t < n; t += kThreads)
            if (cand_p[t] >= p_k) mk += fixed(cand_p[t]);
          uint32_t zc = 0;
          uint32_t tc;
          unsigned long long tm;
          block_scan(sh, zc, mk, tc, tm);
          if (tm >= p_target) {
            float best_v = p_k;
            for (uint32_t t = threadIdx.x; t < n; t += kThreads) {
              const float v = cand_p[t];
              if (v < p_k) continue;
              unsigned long long mv = 0;
              for (uint32_t u = 0; u < n; ++u)
                if (cand_p[u] >= v) mv += fixed(cand_p[u]);
              if (mv >= p_target) best_v = fmaxf(best_v, v);
            }
            float bv = best_v;
            int64_t bi = 0;
            block_argmax(sh, bv, bi);
            cut = bv;
          }
        }
        if (ok) {
          // The race over the surviving candidates (order-independent: larger key, then
          // lower index).
          float best = -INFINITY;
          int64_t best_i = vocab;
          for (uint32_t t = threadIdx.x; t < n; t += kThreads) {
            const float pt = cand_p[t];
            if (!(pt > 0.f && pt >= cut)) continue;
            const int64_t i = cand_i[t];
            const uint4 rnd =
                philox4x32_10(make_uint4(static_cast<uint32_t>(i >> 2), static_cast<uint32_t>(row),
                                         a.offset_lo, a.offset_hi),
                              k0, k1);
            const uint32_t words[4] = {rnd.x, rnd.y, rnd.z, rnd.w};
            const float key = cand_s[t] + gumbel(words[i & 3]);
            if (key > best || (key == best && i < best_i)) {
              best = key;
              best_i = i;
            }
          }
          block_argmax(sh, best, best_i);
          if (threadIdx.x == 0) a.out[row] = best_i < vocab ? best_i : -1;
          return;
        }
      }
    }
    __syncthreads();  // the candidate lists alias the mass histogram of the radix path
  }

  // Passes 2-4: radix selection of the two cutoffs over the bits of p.
  if (threadIdx.x == 0) {
    sh.k_prefix = 0;
    sh.k_rem = static_cast<uint32_t>(top_k);
    sh.k_active = top_k < vocab;
    sh.p_prefix = 0;
    sh.p_rem = p_target;
  }
  constexpr int kShift[3] = {19, 9, 0};
  constexpr int kBits[3] = {12, 10, 9};
  for (int pass = 0; pass < 3; ++pass) {
    const int shift = kShift[pass], bits = kBits[pass];
    const int nbins = 1 << bits;
    for (int b = threadIdx.x; b < nbins; b += kThreads) {
      sh.cnt[b] = 0;
      sh.mass[b] = 0;
    }
    if (threadIdx.x == 0) {
      sh.p_found = 0;
      sh.k_found = 0;
      sh.p_lowest = 0xffffffffu;
    }
    __syncthreads();
    const uint32_t kp = sh.k_prefix, pp = sh.p_prefix;
    const bool use_k = sh.k_active;
    const int above = shift + bits;
    for_each<DT>(a, row, vec, [&](int64_t, float x) {
      const float s = scaled(x);
      if (s == -INFINITY) return;
      const float p = prob(s);
      const uint32_t key = __float_as_uint(p);
      const uint32_t bin = (key >> shift) & (nbins - 1);
      const uint32_t hi = above >= 32 ? 0u : key >> above;
      if (use_k && hi == kp) atomicAdd(&sh.cnt[bin], 1u);
      if (use_p && hi == pp) {
        const unsigned long long fx = static_cast<unsigned long long>(p * kFixedScale + 0.5f);
        if (fx) atomicAdd(&sh.mass[bin], fx);
      }
    });
    __syncthreads();

    // Each thread owns 4 consecutive bins; the suffix above them is the total
    // minus the inclusive prefix of the thread sums.
    const int b0 = threadIdx.x * 4;
    uint32_t c4[4] = {0, 0, 0, 0};
    unsigned long long m4[4] = {0, 0, 0, 0};
    for (int j = 0; j < 4; ++j)
      if (b0 + j < nbins) {
        c4[j] = sh.cnt[b0 + j];
        m4[j] = sh.mass[b0 + j];
      }
    uint32_t csum = c4[0] + c4[1] + c4[2] + c4[3];
    unsigned long long msum = m4[0] + m4[1] + m4[2] + m4[3];
    uint32_t total_c;
    unsigned long long total_m;
    block_scan(sh, csum, msum, total_c, total_m);
    uint32_t c_above = total_c - csum;
    unsigned long long m_above = total_m - msum;
    const uint32_t k_rem = sh.k_rem;
    const unsigned long long p_rem = sh.p_rem;
    for (int j = 3; j >= 0; --j) {
      const uint32_t b = static_cast<uint32_t>(b0 + j);
      if (use_k && c4[j] && c_above < k_rem && c_above + c4[j] >= k_rem) {
        sh.k_prefix = (kp << bits) | b;
        sh.k_rem = k_rem - c_above;
        sh.k_found = 1;
      }
      if (use_p && m4[j] && m_above < p_rem && m_above + m4[j] >= p_rem) {
        sh.p_prefix = (pp << bits) | b;
        sh.p_rem = p_rem - m_above;
        sh.p_found = 1;
      }
      if (use_p && m4[j]) atomicMin(&sh.p_lowest, b);
      c_above += c4[j];
      m_above += m4[j];
    }
    __syncthreads();
    // Fewer than k finite logits: the top-k cutoff keeps everything.
    if (use_k && threadIdx.x == 0 && !sh.k_found) sh.k_active = 0;
    if (use_p && threadIdx.x == 0 && !sh.p_found) {
      // Rounding kept every prefix below the target: keep the whole lowest bin.
      const uint32_t b = sh.p_lowest == 0xffffffffu ? 0u : sh.p_lowest;
      sh.p_prefix = (pp << bits) | b;
      sh.p_rem = sh.mass[b];
    }
    __syncthreads();
  }
  const float cut_k = sh.k_active ? __uint_as_float(sh.k_prefix) : 0.f;
  const float cut_p = use_p ? __uint_as_float(sh.p_prefix) : 0.f;
  const float cut = fmaxf(cut_k, cut_p);

  // Pass 5: exponential race over the survivors.
  bool unused = false;
  float best;
  int64_t best_i;
  race([&](float s) { const float p = prob(s); return p > 0.f && p >= cut; }, unused, best,
       best_i);
  block_argmax(sh, best, best_i);
  if (threadIdx.x == 0) a.out[row] = best_i < vocab ? best_i : -1;
}

}  // namespace
}  // namespace mi355x

using namespace mi355x;

extern "C" const char* mi355x_sample(const void* logits, int64_t rows, int64_t vocab,
                                     int64_t row_stride, int dtype, const float* temperature,
                                     const int32_t* top_k, const float* top_p, uint64_t seed,
                                     uint64_t offset, int64_t* out, void* stream) {
  if (rows < 0 || vocab <= 0 || row_stride < vocab) return set_error("mi355x_sample: bad shape");
  if (vocab >= (int64_t(1) << 32) || rows >= (int64_t(1) << 31))
    return set_error("mi355x_sample: shape too large");
  if (dtype < 0 || dtype > 2)
    return set_error("mi355x_sample: dtype must be 0 (bf16), 1 (fp16) or 2 (fp32)");
  if (rows == 0) return nullptr;
  if (!logits || !temperature || !top_k || !top_p || !out)
    return set_error("mi355x_sample: null pointer");
  SampleArgs a{};
  a.logits = logits;
  a.rows = rows;
  a.vocab = vocab;
  a.stride = row_stride;
  a.temperature = temperature;
  a.top_k = top_k;
  a.top_p = top_p;
  a.seed_lo = static_cast<uint32_t>(seed);
  a.seed_hi = static_cast<uint32_t>(seed >> 32);
  a.offset_lo = static_cast<uint32_t>(offset);
  a.offset_hi = static_cast<uint32_t>(offset >> 32);
  a.out = out;
  const int per_vec = dtype == 2 ? 4 : 8;
  const bool vec = aligned(logits, 16) && row_stride % per_vec == 0;
  auto s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>(rows));
  if (dtype == 0)
    sample_kernel<0><<<grid, dim3(kThreads), 0, s>>>(a, vec);
  else if (dtype == 1)
    sample_kernel<1><<<grid, dim3(kThreads), 0, s>>>(a, vec);
  else
    sample_kernel<2><<<grid, dim3(kThreads), 0, s>>>(a, vec);
  return launch_status("mi355x_sample");
}
