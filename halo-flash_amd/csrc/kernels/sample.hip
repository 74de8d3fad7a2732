// Device-side token sampling with SamplerState semantics (reference src/core/sampling.cpp:494-563 Distribution /
// Sample, 616-700 SampleGreedy / LinearDistribution, 702-842 PrepareSelected; penalties 69-80; RNG 845-863).
//
// One 1024-thread block per row. The reference device kernels (src/kernels/core.hip:1406-2116) weight tokens in
// 2^-40 fixed point so sums are order-independent, and draw a token of the same distribution; this kernel instead
// repeats the CPU's double arithmetic in the CPU's order wherever the kept set is small enough to sort on chip,
// so the draw itself is the CPU's:
//   1. penalized logits in double (the penalized tokens marked in an LDS bitmap, their entries found by binary
//      search in the sorted penalty list), the maximum (ties to the lower token) and the finite count;
//   2. temperature 0: the argmax;
//   3. linear path (top_k == 0, top_p == 1, no min-p floor): weights exp((v - max) / T) zeroed under the min-p
//      threshold, their sum, and the draw walked in token order (each thread owns a contiguous token range; the
//      range holding the uniform is found by a scan of range sums and walked sequentially);
//   4. sorted path: the best min(candidates, 4096) tokens are collected (a 4096-bin histogram of max - v picks a
//      cut; an exact radix select over (value, token) takes over when ties or a dense bin overflow the cap),
//      bitonic-sorted by (value descending, token ascending) in LDS, and top-p, min-p, the weight sum, the zero
//      drop and the draw run over that list in list order on one lane, as the CPU runs them;
//   5. when the kept set reaches past the sorted 4096 (a flat row with a loose top-p or a min-p floor), the cut
//      and the draw are radix selects over the whole row on 2^-40 fixed-point weights (integer sums, so two runs
//      agree bit for bit); the nonzero count stays exact in double. Only this path can draw differently from the
//      CPU, and only when the uniform falls within rounding of a boundary.
// Every reduction runs in a fixed order, so a row's result never depends on timing.
#include "common.h"
#include "halo_sample.h"

namespace halo::sample {

constexpr std::uint32_t kThreads = 1024;
constexpr std::uint32_t kWaves = kThreads / kWave;
constexpr std::uint32_t kCap = 4096;   // candidates sorted on chip
constexpr std::uint32_t kBins = 4096;  // histogram of max - v, bins 1/64 wide, the last one open-ended
constexpr double kFix = 1099511627776.0;  // 2^40
constexpr std::uint64_t kNoBound = ~0ull;

struct Lds {
  union {
    std::uint32_t bitmap[HALO_SAMPLE_MAX_VOCAB / 32];
    double w[kCap];
  } a;
  union {
    std::uint32_t hist[kBins];
    struct {
      std::uint32_t cnt[256];
      unsigned long long mass[256];
    } radix;
  } b;
  std::uint64_t key[kCap];
  std::uint32_t tok[kCap];
  double rd[kWaves];
  std::uint32_t ru[kWaves];
  unsigned long long rq[kWaves];
  std::uint64_t bq[4];
  std::uint32_t bu[8];
  double bd[4];
};

// Ascending order of DescKey = descending value; +0 and -0 compare equal, as on the CPU.
__device__ __forceinline__ std::uint64_t DescKey(double d) {
  if (d == 0.0) d = 0.0;
  const std::uint64_t b = static_cast<std::uint64_t>(__double_as_longlong(d));
  const std::uint64_t k = (b >> 63) ? ~b : (b | (1ull << 63));
  return ~k;
}
__device__ __forceinline__ double KeyValue(std::uint64_t kd) {
  const std::uint64_t k = ~kd;
  const std::uint64_t b = (k >> 63) ? (k & ~(1ull << 63)) : ~k;
  return __longlong_as_double(static_cast<long long>(b));
}

// xorshift64* (Vigna; the reference's NextRandom / Uniform, sampling.cpp:845-863): a zero state is replaced by
// the 64-bit golden-ratio constant; the uniform takes the top 53 bits.
__device__ __forceinline__ std::uint64_t NextRandom(std::uint64_t* state) {
  std::uint64_t v = *state ? *state : 0x9e3779b97f4a7c15ull;
  v ^= v >> 12;
  v ^= v << 25;
  v ^= v >> 27;
  *state = v;
  return v * 0x2545f4914f6cdd1dull;
}
__device__ __forceinline__ double Uniform(std::uint64_t* state) {
  return static_cast<double>(NextRandom(state) >> 11) * 0x1.0p-53;
}

__device__ __forceinline__ double Penalize(double l, const HaloSampleParams& p, const HaloPenalty& e) {
  if (e.repeated && p.repeat_penalty != 1.0f) l = l <= 0 ? l * p.repeat_penalty : l / p.repeat_penalty;
  l -= static_cast<double>(p.frequency_penalty) * e.generated_count;
  if (e.generated_count != 0) l -= p.presence_penalty;
  return l;
}

// ---- block-wide reductions in a fixed order (every thread calls; every thread gets the result) --------------
__device__ double BlockSumD(double v, Lds& s) {
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  if (threadIdx.x % kWave == 0) s.rd[threadIdx.x / kWave] = v;
  __syncthreads();
  double r = 0.0;
  for (std::uint32_t i = 0; i < kWaves; ++i) r += s.rd[i];
  __syncthreads();
  return r;
}
__device__ std::uint32_t BlockSumU(std::uint32_t v, Lds& s) {
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  if (threadIdx.x % kWave == 0) s.ru[threadIdx.x / kWave] = v;
  __syncthreads();
  std::uint32_t r = 0;
  for (std::uint32_t i = 0; i < kWaves; ++i) r += s.ru[i];
  __syncthreads();
  return r;
}
__device__ unsigned long long BlockSumQ(unsigned long long v, Lds& s) {
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  if (threadIdx.x % kWave == 0) s.rq[threadIdx.x / kWave] = v;
  __syncthreads();
  unsigned long long r = 0;
  for (std::uint32_t i = 0; i < kWaves; ++i) r += s.rq[i];
  __syncthreads();
  return r;
}
// Exclusive prefix over threads in thread order; *total = the block total.
template <typename T>
__device__ T BlockExclScan(T v, T* wave_tot, T* total) {
  const std::uint32_t lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  T inc = v;
  for (int o = 1; o < kWave; o <<= 1) {
    const T n = __shfl_up(inc, o, kWave);
    if (lane >= static_cast<std::uint32_t>(o)) inc += n;
  }
  T exc = __shfl_up(inc, 1, kWave);
  if (lane == 0) exc = 0;
  if (lane == kWave - 1) wave_tot[w] = inc;
  __syncthreads();
  T base = 0, tot = 0;
  for (std::uint32_t i = 0; i < kWaves; ++i) {
    if (i < w) base += wave_tot[i];
    tot += wave_tot[i];
  }
  __syncthreads();
  *total = tot;
  return base + exc;
}
// Smallest (key, token) pair over the block (the best candidate when keys are DescKeys).
__device__ void BlockMinPair(std::uint64_t& k, std::uint32_t& t, Lds& s) {
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const std::uint64_t ok = __shfl_xor(k, o, kWave);
    const std::uint32_t ot = __shfl_xor(t, o, kWave);
    if (ok < k || (ok == k && ot < t)) {
      k = ok;
      t = ot;
    }
  }
  if (threadIdx.x % kWave == 0) {
    s.rq[threadIdx.x / kWave] = k;
    s.ru[threadIdx.x / kWave] = t;
  }
  __syncthreads();
  k = s.rq[0];
  t = s.ru[0];
  for (std::uint32_t i = 1; i < kWaves; ++i)
    if (s.rq[i] < k || (s.rq[i] == k && s.ru[i] < t)) {
      k = s.rq[i];
      t = s.ru[i];
    }
  __syncthreads();
}

__device__ __forceinline__ bool Within(std::uint64_t kd, std::uint32_t t, std::uint64_t lk, std::uint32_t lt) {
  return kd < lk || (kd == lk && t <= lt);
}

// Radix select over (DescKey, token), 8 digits of the key then 8 + 8 + 2 bits of the token: the first element e in
// ascending order among finite elements within (lk, lt) whose inclusive cumulative weight reaches `target`
// (weight 1 per element when fx is null, fx[i] otherwise). Returns false when the total stays below the target.
// *before_n / *before_m: count and weight of the elements ahead of e.
__device__ bool Select(const double* __restrict__ val, const unsigned long long* __restrict__ fx, std::uint32_t V,
                       unsigned long long target, std::uint64_t lk, std::uint32_t lt, Lds& s, std::uint64_t* ek,
                       std::uint32_t* et, unsigned long long* before_n, unsigned long long* before_m) {
  std::uint64_t kpre = 0, kmask = 0;
  std::uint32_t tpre = 0, tmask = 0;
  unsigned long long rem = target, bn = 0, bm = 0;
  bool found = true;
  for (int pass = 0; pass < 11; ++pass) {
    int shift;
    bool on_key;
    std::uint32_t width;
    if (pass < 8) {
      on_key = true;
      shift = 56 - 8 * pass;
      width = 8;
    } else {
      on_key = false;
      shift = pass == 8 ? 10 : (pass == 9 ? 2 : 0);
      width = pass == 10 ? 2 : 8;
    }
    const std::uint32_t dmask = (1u << width) - 1;
    for (std::uint32_t i = threadIdx.x; i < 256; i += kThreads) {
      s.b.radix.cnt[i] = 0;
      s.b.radix.mass[i] = 0;
    }
    __syncthreads();
    for (std::uint32_t i = threadIdx.x; i < V; i += kThreads) {
      const double v = val[i];
      if (v == -INFINITY) continue;
      const std::uint64_t kd = DescKey(v);
      if (!Within(kd, i, lk, lt) || (kd & kmask) != kpre || (i & tmask) != tpre) continue;
      const std::uint32_t d = on_key ? static_cast<std::uint32_t>(kd >> shift) & dmask : (i >> shift) & dmask;
      atomicAdd(&s.b.radix.cnt[d], 1u);
      if (fx) atomicAdd(&s.b.radix.mass[d], fx[i]);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      std::uint32_t pick = 0xFFFFFFFFu;
      for (std::uint32_t d = 0; d <= dmask; ++d) {
        const std::uint32_t c = s.b.radix.cnt[d];
        if (c == 0) continue;
        const unsigned long long m = fx ? s.b.radix.mass[d] : c;
        if (rem <= m) {
          pick = d;
          break;
        }
        rem -= m;
        bn += c;
        bm += s.b.radix.mass[d];
      }
      s.bu[0] = pick;
      s.bq[0] = rem;
      s.bq[1] = bn;
      s.bq[2] = bm;
    }
    __syncthreads();
    const std::uint32_t pick = s.bu[0];
    rem = s.bq[0];
    bn = s.bq[1];
    bm = s.bq[2];
    __syncthreads();
    if (pick == 0xFFFFFFFFu) {
      found = false;
      break;
    }
    if (on_key) {
      kpre |= static_cast<std::uint64_t>(pick) << shift;
      kmask |= static_cast<std::uint64_t>(dmask) << shift;
    } else {
      tpre |= pick << shift;
      tmask |= dmask << shift;
    }
  }
  *ek = kpre;
  *et = tpre;
  *before_n = bn;
  *before_m = bm;
  return found;
}

__device__ void Finish(HaloSampleOut* out, std::uint32_t token, std::uint32_t live, std::uint64_t rng) {
  if (threadIdx.x == 0) {
    HaloSampleOut o;
    o.token = token;
    o.live = live;
    o.rng = rng;
    *out = o;
  }
}

}  // namespace halo::sample

// One draw per row. logits [rows][row_stride] fp32 (vocab tokens each); params [rows]; penalties
// [rows][pen_stride] (params[r].n_penalties used, sorted by token); vals [rows][vocab] double and fx
// [rows][vocab] u64 are workspace; out [rows]. Block 1024, grid rows.
extern "C" __global__ void __launch_bounds__(1024)
    halo_sample_rows(const float* __restrict__ logits, std::uint64_t row_stride,
                     const HaloSampleParams* __restrict__ params, const HaloPenalty* __restrict__ penalties,
                     std::uint32_t pen_stride, std::uint32_t V, double* __restrict__ vals,
                     unsigned long long* __restrict__ fxs, HaloSampleOut* __restrict__ outs) {
  using namespace halo::sample;
  __shared__ Lds s;
  const std::uint32_t row = blockIdx.x, t = threadIdx.x;
  const HaloSampleParams p = params[row];
  const float* x = logits + row * row_stride;
  const HaloPenalty* pen = penalties + static_cast<std::size_t>(row) * pen_stride;
  double* val = vals + static_cast<std::size_t>(row) * V;
  unsigned long long* fx = fxs + static_cast<std::size_t>(row) * V;
  HaloSampleOut* out = outs + row;
  std::uint64_t rng = p.rng;

  const bool bad = p.vocab != V || V == 0 || V > HALO_SAMPLE_MAX_VOCAB || p.n_penalties > pen_stride ||
                   p.n_penalties > HALO_SAMPLE_MAX_PENALTIES || !isfinite(p.temperature) || p.temperature < 0.0f ||
                   !(p.top_p >= 0.0f && p.top_p <= 1.0f) || !(p.min_p >= 0.0f && p.min_p <= 1.0f) ||
                   !isfinite(p.repeat_penalty) || !(p.repeat_penalty > 0.0f) || !isfinite(p.frequency_penalty) ||
                   !isfinite(p.presence_penalty) || p.top_k > 0x7FFFFFFFu;
  if (bad) {
    Finish(out, HALO_SAMPLE_BAD_PARAMS, 0, rng);
    return;
  }

  // 1. penalized values, maximum, finite count
  const std::uint32_t npen = p.n_penalties;
  if (npen) {
    for (std::uint32_t i = t; i < (V + 31) / 32; i += kThreads) s.a.bitmap[i] = 0;
    __syncthreads();
    for (std::uint32_t j = t; j < npen; j += kThreads) {
      const std::uint32_t tk = pen[j].token;
      if (tk < V) atomicOr(&s.a.bitmap[tk >> 5], 1u << (tk & 31));
    }
    __syncthreads();
  }
  std::uint64_t best_k = kNoBound;
  std::uint32_t best_t = 0xFFFFFFFFu, nf = 0;
  for (std::uint32_t i = t; i < V; i += kThreads) {
    const float l = x[i];
    double a = -INFINITY;
    if (isfinite(l)) {
      a = l;
      if (npen && (s.a.bitmap[i >> 5] >> (i & 31)) & 1u) {
        std::uint32_t lo = 0, hi = npen;
        while (lo < hi) {
          const std::uint32_t mid = (lo + hi) / 2;
          if (pen[mid].token < i) lo = mid + 1;
          else hi = mid;
        }
        if (lo < npen && pen[lo].token == i) a = Penalize(a, p, pen[lo]);  // an unsorted list finds nothing
      }
      ++nf;
      const std::uint64_t kd = DescKey(a);
      if (kd < best_k) {  // ascending i per thread: the first maximum wins
        best_k = kd;
        best_t = i;
      }
    }
    val[i] = a;
  }
  nf = BlockSumU(nf, s);
  BlockMinPair(best_k, best_t, s);
  if (nf == 0) {
    Finish(out, HALO_SAMPLE_NO_FINITE, 0, rng);
    return;
  }
  if (p.temperature == 0.0f) {
    Finish(out, best_t, 1, rng);
    return;
  }
  const double M = KeyValue(best_k);
  const double T = p.temperature;
  const std::uint32_t floor_keep = p.min_keep > 1 ? p.min_keep : 1;

  // 2. linear path: token order
  if (p.top_k == 0 && p.top_p == 1.0f && !(p.min_p > 0.0f && p.min_keep > 1)) {
    const double thr = p.min_p > 0.0f ? M + T * log(static_cast<double>(p.min_p)) : -INFINITY;
    const std::uint32_t per = (V + kThreads - 1) / kThreads, lo = min(V, t * per), hi = min(V, lo + per);
    double part = 0.0;
    for (std::uint32_t i = lo; i < hi; ++i) {
      const double a = val[i];
      const double w = (a != -INFINITY && a >= thr) ? exp((a - M) / T) : 0.0;
      val[i] = w;
      part += w;
    }
    const double total = BlockSumD(part, s);
    std::uint32_t nz = 0, last = 0;
    double ps = 0.0;
    for (std::uint32_t i = lo; i < hi; ++i) {
      const double v = val[i] / total;
      if (v != 0.0) {
        ++nz;
        last = i + 1;
        ps += v;
      }
    }
    const std::uint32_t live = BlockSumU(nz, s);
    std::uint64_t lk = ~static_cast<std::uint64_t>(last);  // the largest index with a nonzero weight
    std::uint32_t lt = 0;
    BlockMinPair(lk, lt, s);
    const std::uint32_t last_nz = static_cast<std::uint32_t>(~lk) - 1;
    if (live == 1) {
      Finish(out, last_nz, 1, rng);
      return;
    }
    const double u = Uniform(&rng);
    double tot;
    const double ex = BlockExclScan(ps, s.rd, &tot);
    if (t == 0) s.bu[1] = 0xFFFFFFFFu;
    __syncthreads();
    if (ps > 0.0 && u >= ex && u < ex + ps) {
      double r = u - ex;
      for (std::uint32_t i = lo; i < hi; ++i) {
        const double v = val[i] / total;
        if (v == 0.0) continue;
        r -= v;
        if (r < 0.0) {
          atomicMin(&s.bu[1], i);
          break;
        }
      }
    }
    __syncthreads();
    const std::uint32_t pick = s.bu[1];
    Finish(out, pick == 0xFFFFFFFFu ? last_nz : pick, live, rng);
    return;
  }

  // 3. sorted path: collect the best Rc candidates
  const std::uint64_t keep_cfg =
      p.top_k > 0 ? min(static_cast<std::uint64_t>(V), static_cast<std::uint64_t>(max(p.top_k, floor_keep)))
                  : static_cast<std::uint64_t>(V);
  const std::uint32_t K0 = static_cast<std::uint32_t>(min(static_cast<std::uint64_t>(nf), keep_cfg));
  const std::uint32_t Rc = min(K0, kCap);
  const bool has_full = p.top_k == 0 && p.top_p < 1.0f && V > 1024;
  double full_sum = 0.0;
  if (has_full) {
    double part = 0.0;
    for (std::uint32_t i = t; i < V; i += kThreads) {
      const double a = val[i];
      if (a != -INFINITY) part += exp((a - M) / T);
    }
    full_sum = BlockSumD(part, s);
  }
  for (std::uint32_t i = t; i < kBins; i += kThreads) s.b.hist[i] = 0;
  __syncthreads();
  for (std::uint32_t i = t; i < V; i += kThreads) {
    const double a = val[i];
    if (a == -INFINITY) continue;
    const double d = M - a;
    const std::uint32_t bin = d < 64.0 ? static_cast<std::uint32_t>(d * 64.0) : kBins - 1;
    atomicAdd(&s.b.hist[bin], 1u);
  }
  __syncthreads();
  {
    std::uint32_t c4 = 0;
    for (std::uint32_t j = 0; j < kBins / kThreads; ++j) c4 += s.b.hist[t * (kBins / kThreads) + j];
    std::uint32_t tot;
    std::uint32_t base = BlockExclScan(c4, s.ru, &tot);
    for (std::uint32_t j = 0; j < kBins / kThreads; ++j) {
      const std::uint32_t h = s.b.hist[t * (kBins / kThreads) + j];
      if (base < Rc && base + h >= Rc) {
        s.bu[2] = t * (kBins / kThreads) + j;
        s.bu[3] = base + h;
      }
      base += h;
    }
    if (t == 0) s.bu[4] = 0;
    __syncthreads();
  }
  const std::uint32_t cut_bin = s.bu[2], cut_count = s.bu[3];
  if (cut_count <= kCap) {
    for (std::uint32_t i = t; i < V; i += kThreads) {
      const double a = val[i];
      if (a == -INFINITY) continue;
      const double d = M - a;
      const std::uint32_t bin = d < 64.0 ? static_cast<std::uint32_t>(d * 64.0) : kBins - 1;
      if (bin <= cut_bin) {
        const std::uint32_t slot = atomicAdd(&s.bu[4], 1u);
        s.key[slot] = DescKey(a);
        s.tok[slot] = i;
      }
    }
  } else {
    // exact: the Rc-th best (value, token) by radix select, then everything up to it
    std::uint64_t ck;
    std::uint32_t ct;
    unsigned long long bn, bm;
    Select(val, nullptr, V, Rc, kNoBound, 0xFFFFFFFFu, s, &ck, &ct, &bn, &bm);
    for (std::uint32_t i = t; i < V; i += kThreads) {
      const double a = val[i];
      if (a == -INFINITY) continue;
      const std::uint64_t kd = DescKey(a);
      if (Within(kd, i, ck, ct)) {
        const std::uint32_t slot = atomicAdd(&s.bu[4], 1u);
        s.key[slot] = kd;
        s.tok[slot] = i;
      }
    }
  }
  __syncthreads();
  const std::uint32_t n = s.bu[4];
  std::uint32_t P = 1;
  while (P < n) P <<= 1;
  for (std::uint32_t i = n + t; i < P; i += kThreads) {
    s.key[i] = kNoBound;
    s.tok[i] = 0xFFFFFFFFu;
  }
  __syncthreads();
  for (std::uint32_t k = 2; k <= P; k <<= 1) {
    for (std::uint32_t j = k >> 1; j > 0; j >>= 1) {
      for (std::uint32_t i = t; i < P; i += kThreads) {
        const std::uint32_t l = i ^ j;
        if (l > i) {
          const std::uint64_t ki = s.key[i], kl = s.key[l];
          const std::uint32_t ti = s.tok[i], tl = s.tok[l];
          const bool greater = ki > kl || (ki == kl && ti > tl);
          if (((i & k) == 0) == greater) {
            s.key[i] = kl;
            s.key[l] = ki;
            s.tok[i] = tl;
            s.tok[l] = ti;
          }
        }
      }
      __syncthreads();
    }
  }
  // weights of the sorted list
  for (std::uint32_t i = t; i < Rc; i += kThreads) s.a.w[i] = exp((KeyValue(s.key[i]) - M) / T);
  __syncthreads();
  // 4. top-p, min-p and the weight sum in list order, one lane (the CPU's order)
  if (t == 0) {
    std::uint32_t keep = K0;
    const std::uint32_t minimum = min(K0, floor_keep);
    bool large = false;
    if (p.top_p < 1.0f && K0 > 1) {
      double sum = full_sum;
      if (!has_full) {
        if (K0 > Rc) {
          large = true;
        } else {
          sum = 0.0;
          for (std::uint32_t i = 0; i < K0; ++i) sum += s.a.w[i];
        }
      }
      if (!large) {
        const double target = static_cast<double>(p.top_p) * sum;
        double cumulative = 0.0;
        std::uint32_t k = 0;
        while (k < K0) {
          if (k == Rc) {
            large = true;
            break;
          }
          cumulative += s.a.w[k];
          ++k;
          if (k >= minimum && cumulative >= target) break;
        }
        keep = k;
      }
    }
    if (!large && p.min_p > 0.0f && keep > 1) {
      const double thr = M + T * log(static_cast<double>(p.min_p));
      std::uint32_t k = 0;
      while (k < keep && k < Rc && KeyValue(s.key[k]) >= thr) ++k;
      if (k == Rc && Rc < keep) large = true;
      else keep = min(keep, max(k, minimum));
    }
    if (!large && keep > Rc) large = true;
    double total = 0.0;
    if (!large)
      for (std::uint32_t i = 0; i < keep; ++i) total += s.a.w[i];
    s.bu[5] = keep;
    s.bu[6] = large;
    s.bd[0] = total;
  }
  __syncthreads();
  const bool large = s.bu[6] != 0;
  if (!large) {
    const std::uint32_t keep = s.bu[5];
    const double total = s.bd[0];
    std::uint32_t nz = 0, last = 0;
    for (std::uint32_t i = t; i < keep; i += kThreads) {
      const double v = s.a.w[i] / total;
      s.a.w[i] = v;
      if (v != 0.0) {
        ++nz;
        last = max(last, i + 1);
      }
    }
    const std::uint32_t live = BlockSumU(nz, s);
    std::uint64_t lk = ~static_cast<std::uint64_t>(last);
    std::uint32_t lt = 0;
    BlockMinPair(lk, lt, s);
    const std::uint32_t last_nz = static_cast<std::uint32_t>(~lk) - 1;
    if (t == 0) {
      std::uint32_t token = s.tok[last_nz];
      if (live > 1) {
        double r = Uniform(&rng);
        for (std::uint32_t i = 0; i < keep; ++i) {
          r -= s.a.w[i];
          if (r < 0.0) {
            token = s.tok[i];
            break;
          }
        }
      }
      Finish(out, token, live, rng);
    }
    return;
  }

  // 5. the kept set reaches past the sorted list: fixed-point selects over the whole row
  for (std::uint32_t i = t; i < V; i += kThreads) {
    const double a = val[i];
    fx[i] = a == -INFINITY ? 0ull : static_cast<unsigned long long>(exp((a - M) / T) * kFix);
  }
  __syncthreads();
  std::uint64_t lk0 = kNoBound;
  std::uint32_t lt0 = 0xFFFFFFFFu;
  unsigned long long bn, bm;
  if (K0 < nf) Select(val, nullptr, V, K0, kNoBound, 0xFFFFFFFFu, s, &lk0, &lt0, &bn, &bm);
  const std::uint32_t minimum = min(K0, floor_keep);
  std::uint32_t keep = K0;
  if (p.top_p < 1.0f && K0 > 1) {
    unsigned long long part = 0;
    for (std::uint32_t i = t; i < V; i += kThreads) {
      const double a = val[i];
      if (a != -INFINITY && Within(DescKey(a), i, lk0, lt0)) part += fx[i];
    }
    const unsigned long long sum = BlockSumQ(part, s);
    const unsigned long long target =
        static_cast<unsigned long long>(ceil(static_cast<double>(p.top_p) * static_cast<double>(sum)));
    std::uint64_t ek;
    std::uint32_t et;
    if (Select(val, fx, V, target, lk0, lt0, s, &ek, &et, &bn, &bm))
      keep = max(static_cast<std::uint32_t>(bn) + 1, minimum);
  }
  if (p.min_p > 0.0f && keep > 1) {
    const double thr = M + T * log(static_cast<double>(p.min_p));
    std::uint32_t c = 0;
    for (std::uint32_t i = t; i < V; i += kThreads) {
      const double a = val[i];
      if (a != -INFINITY && a >= thr) ++c;
    }
    c = BlockSumU(c, s);
    keep = min(keep, max(c, minimum));
  }
  std::uint64_t lk = kNoBound;
  std::uint32_t lt = 0xFFFFFFFFu;
  if (keep < nf) Select(val, nullptr, V, keep, kNoBound, 0xFFFFFFFFu, s, &lk, &lt, &bn, &bm);
  double part = 0.0;
  unsigned long long qpart = 0;
  for (std::uint32_t i = t; i < V; i += kThreads) {
    const double a = val[i];
    if (a != -INFINITY && Within(DescKey(a), i, lk, lt)) {
      part += exp((a - M) / T);
      qpart += fx[i];
    }
  }
  const double total = BlockSumD(part, s);
  const unsigned long long qtotal = BlockSumQ(qpart, s);
  std::uint32_t nz = 0;
  std::uint64_t last_k = 0;  // the worst kept (key, token) with a nonzero weight: max order = min of complements
  std::uint32_t last_t = 0;
  std::uint64_t nk = kNoBound;
  std::uint32_t nt = 0xFFFFFFFFu;
  for (std::uint32_t i = t; i < V; i += kThreads) {
    const double a = val[i];
    if (a == -INFINITY) continue;
    const std::uint64_t kd = DescKey(a);
    if (!Within(kd, i, lk, lt) || exp((a - M) / T) / total == 0.0) continue;
    ++nz;
    if (~kd < nk || (~kd == nk && ~i < nt)) {
      nk = ~kd;
      nt = ~i;
    }
  }
  const std::uint32_t live = BlockSumU(nz, s);
  BlockMinPair(nk, nt, s);
  last_k = ~nk;
  last_t = ~nt;
  (void)last_k;
  if (live == 1) {
    Finish(out, best_t, 1, rng);
    return;
  }
  const double u = Uniform(&rng);
  const unsigned long long target = static_cast<unsigned long long>(floor(u * static_cast<double>(qtotal))) + 1;
  std::uint64_t ek;
  std::uint32_t et;
  const bool found = Select(val, fx, V, target, lk, lt, s, &ek, &et, &bn, &bm);
  Finish(out, found ? et : last_t, live, rng);
}
