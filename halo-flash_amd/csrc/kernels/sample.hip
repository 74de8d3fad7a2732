// Device-side token sampling with SamplerState semantics (reference src/core/sampling.cpp:494-563 Distribution /
// Sample, 616-700 SampleGreedy / LinearDistribution, 702-842 PrepareSelected; penalties 69-80; RNG 845-863).
//
// The reference device kernels (src/kernels/core.hip:1406-2116) weight tokens in 2^-40 fixed point so sums are
// order-independent, and draw a token of the same distribution; these kernels instead repeat the CPU's double
// arithmetic in the CPU's order wherever the kept set is small enough to sort on chip, so the draw itself is the
// CPU's. Four launches per call; the first three spread the vocabulary over blocks of 4096 tokens, the last runs
// one 1024-thread block per row:
//   1. prep: penalized logits in double (penalized tokens marked in an LDS bitmap per slice, their entries found
//      by binary search in the sorted penalty list), each slice's maximum (ties to the lower token) and finite
//      count;
//   2. weights: linear path (top_k == 0, top_p == 1, no min-p floor): weights exp((v - max) / T), zeroed under the
//      min-p threshold, with per-slice sums, nonzero counts, last nonzero index and least nonzero weight; sorted
//      path: a 4096-bin histogram of max - v (bins 1/64 wide) and, for top-p without top-k over more than 1024
//      tokens, the per-slice weight sums;
//   3. collect (sorted path): the bins that hold the best min(candidates, 4096) tokens, or the full bins before
//      them, are cut from the histogram and their tokens appended to a candidate list;
//   4. final: temperature 0 takes the argmax; the linear path finds the slice, then the 4-token range, holding the
//      uniform and walks it in token order; the sorted path orders the candidates by (value descending, token
//      ascending) in LDS: counted again over 4096 fine bins spanning the collected range, scattered to their bin's
//      place and ranked within it (a bitonic sort when a bin overflows; an exact radix select over (value, token)
//      replaces the histogram cut when ties overflow it), and runs top-p, min-p, the weight sum, the zero drop and
//      the draw over that list in list order on one lane, as the CPU runs them (one add per element: the running
//      sums are monotone, so only a chunk's last sum is tested); when the kept set reaches past the sorted
//      candidates (a flat row with a loose top-p or a min-p floor), the cut and the draw are radix selects over the
//      whole row on 2^-40 fixed-point weights (integer sums, so runs agree bit for bit) and the nonzero count
//      stays exact in double.
// Only sums formed across slices or threads (the linear path's total, the full top-p sum, the fixed-point path)
// differ from the CPU's sequential sums, by rounding; they move a draw only when the uniform falls within rounding
// of a CDF boundary. Every reduction runs in a fixed order, so a row's result never depends on timing.
#include "common.h"
#include "halo_sample.h"
#include "sample_layout.h"

namespace halo::sample {

constexpr std::uint32_t kThreads = 1024;
constexpr std::uint32_t kWaves = kThreads / kWave;
constexpr std::uint32_t kCap = kSampleCap;   // candidates sorted on chip
constexpr std::uint32_t kBins = kSampleBins;  // histogram of max - v, bins 1/64 wide, the last one open-ended
static_assert((HALO_SAMPLE_MAX_VOCAB + kSampleSlice - 1) / kSampleSlice <= kWave,
              "one wave holds every slice's partials");
constexpr double kFix = 1099511627776.0;  // 2^40
constexpr std::uint64_t kNoBound = ~0ull;

struct Lds {
  union alignas(16) {
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
  double xd;  // wave-0 reductions of the per-slice partials, broadcast
  std::uint32_t xu;
  unsigned long long xq[2];
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
template <typename T>
__device__ T WaveSum(T v) {
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
// Smallest (key, token) pair over the wave.
__device__ void WaveMinPair(std::uint64_t& k, std::uint32_t& t) {
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const std::uint64_t ok = __shfl_xor(k, o, kWave);
    const std::uint32_t ot = __shfl_xor(t, o, kWave);
    if (ok < k || (ok == k && ot < t)) {
      k = ok;
      t = ot;
    }
  }
}
template <typename T>
__device__ T BlockSum(T v, T* red) {
  v = WaveSum(v);
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  T r = 0;
  for (std::uint32_t i = 0; i < blockDim.x / kWave; ++i) r += red[i];
  __syncthreads();
  return r;
}
__device__ double BlockSumD(double v, Lds& s) { return BlockSum(v, s.rd); }
__device__ std::uint32_t BlockSumU(std::uint32_t v, Lds& s) { return BlockSum(v, s.ru); }
__device__ unsigned long long BlockSumQ(unsigned long long v, Lds& s) { return BlockSum(v, s.rq); }
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
  for (std::uint32_t i = 0; i < blockDim.x / kWave; ++i) {
    if (i < w) base += wave_tot[i];
    tot += wave_tot[i];
  }
  __syncthreads();
  *total = tot;
  return base + exc;
}
// Smallest (key, token) pair over the block (the best candidate when keys are DescKeys).
__device__ void BlockMinPair(std::uint64_t& k, std::uint32_t& t, unsigned long long* rk, std::uint32_t* rt) {
  WaveMinPair(k, t);
  if (threadIdx.x % kWave == 0) {
    rk[threadIdx.x / kWave] = k;
    rt[threadIdx.x / kWave] = t;
  }
  __syncthreads();
  k = rk[0];
  t = rt[0];
  for (std::uint32_t i = 1; i < blockDim.x / kWave; ++i)
    if (rk[i] < k || (rk[i] == k && rt[i] < t)) {
      k = rk[i];
      t = rt[i];
    }
  __syncthreads();
}
__device__ void BlockMinPair(std::uint64_t& k, std::uint32_t& t, Lds& s) { BlockMinPair(k, t, s.rq, s.ru); }

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

__device__ __forceinline__ bool BadParams(const HaloSampleParams& p, std::uint32_t V, std::uint32_t pen_stride) {
  return p.vocab != V || V == 0 || V > HALO_SAMPLE_MAX_VOCAB || p.n_penalties > pen_stride ||
         p.n_penalties > HALO_SAMPLE_MAX_PENALTIES || !isfinite(p.temperature) || p.temperature < 0.0f ||
         !(p.top_p >= 0.0f && p.top_p <= 1.0f) || !(p.min_p >= 0.0f && p.min_p <= 1.0f) ||
         !isfinite(p.repeat_penalty) || !(p.repeat_penalty > 0.0f) || !isfinite(p.frequency_penalty) ||
         !isfinite(p.presence_penalty) || p.top_k > 0x7FFFFFFFu;
}
__device__ __forceinline__ bool LinearPath(const HaloSampleParams& p) {
  return p.top_k == 0 && p.top_p == 1.0f && !(p.min_p > 0.0f && p.min_keep > 1);
}
__device__ __forceinline__ std::uint32_t Bin(double M, double a) {
  const double d = M - a;
  return d < 64.0 ? static_cast<std::uint32_t>(d * 64.0) : kBins - 1;
}

// Views of one launch's workspace.
struct Ws {
  double* val;
  unsigned long long* fx;
  unsigned long long* pkey;
  std::uint32_t *ptok, *pnf;
  double* psum;
  std::uint32_t *pnz, *plast;
  double* pminw;
  std::uint32_t* hist;
  unsigned long long* ckey;
  std::uint32_t *ctok, *cn;
};
__device__ __forceinline__ Ws Carve(void* base, std::uint32_t rows, std::uint32_t V) {
  const Layout l = MakeLayout(rows, V);
  char* b = static_cast<char*>(base);
  Ws w;
  w.val = reinterpret_cast<double*>(b + l.val);
  w.fx = reinterpret_cast<unsigned long long*>(b + l.fx);
  w.pkey = reinterpret_cast<unsigned long long*>(b + l.pkey);
  w.ptok = reinterpret_cast<std::uint32_t*>(b + l.ptok);
  w.pnf = reinterpret_cast<std::uint32_t*>(b + l.pnf);
  w.psum = reinterpret_cast<double*>(b + l.psum);
  w.pnz = reinterpret_cast<std::uint32_t*>(b + l.pnz);
  w.plast = reinterpret_cast<std::uint32_t*>(b + l.plast);
  w.pminw = reinterpret_cast<double*>(b + l.pminw);
  w.hist = reinterpret_cast<std::uint32_t*>(b + l.hist);
  w.ckey = reinterpret_cast<unsigned long long*>(b + l.ckey);
  w.ctok = reinterpret_cast<std::uint32_t*>(b + l.ctok);
  w.cn = reinterpret_cast<std::uint32_t*>(b + l.cn);
  return w;
}

// The row's maximum (as DescKey, ties to the lower token) and finite count from the per-block partials, in block
// order; every thread gets them.
struct RowMax {
  std::uint64_t key;
  std::uint32_t tok, nf;
};
// nb <= kWave (vocabularies up to 64 slices): wave 0 holds every slice's partials and reduces them with the block
// reductions' shuffle trees (the other waves would add only zeros and neutral pairs, so the results are those of the
// block forms), then one broadcast through LDS.
__device__ RowMax ReduceParts(const Ws& w, std::uint32_t row, std::uint32_t nb, unsigned long long* rk,
                              std::uint32_t* rt, std::uint32_t* ru) {
  if (threadIdx.x < kWave) {
    std::uint64_t k = kNoBound;
    std::uint32_t tk = 0xFFFFFFFFu, nf = 0;
    if (threadIdx.x < nb) {
      const std::size_t o = static_cast<std::size_t>(row) * nb + threadIdx.x;
      k = w.pkey[o];
      tk = w.ptok[o];
      nf = w.pnf[o];
    }
    nf = WaveSum(nf);
    WaveMinPair(k, tk);
    if (threadIdx.x == 0) {
      rk[0] = k;
      rt[0] = tk;
      ru[1] = nf;  // callers may pass one array as rt and ru
    }
  }
  __syncthreads();
  const RowMax m{rk[0], rt[0], ru[1]};
  __syncthreads();
  return m;
}

// Sequential double chains in list order on one lane (they must stay left-to-right to round as the CPU does), over
// the on-chip candidate list w[kCap] (n <= kCap). Chunks of 16 are read whole as 8 double2 (in bounds: a chunk starts
// below n <= kCap, a multiple of 16); full chunks add without per-entry bounds tests, the last one selects entries
// past n to +0.0 (adding +0.0 to a sum of non-negative weights leaves it unchanged), and a chunk's tests are folded
// into a bit mask off the add chain, so an element costs about one add latency.
struct SeqChunk {
  double v[16];
};
__device__ __forceinline__ SeqChunk SeqLoad(const double* w, std::uint32_t k0, std::uint32_t n) {
  const double2* p = reinterpret_cast<const double2*>(w + k0);
  SeqChunk c;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const double2 d = p[j];
    c.v[2 * j] = d.x;
    c.v[2 * j + 1] = d.y;
  }
  if (k0 + 16 > n) {
#pragma unroll
    for (int j = 0; j < 16; ++j) c.v[j] = k0 + j < n ? c.v[j] : 0.0;
  }
  return c;
}
__device__ double SeqSum(const double* w, std::uint32_t n) {
  double sum = 0.0;
  for (std::uint32_t k0 = 0; k0 < n; k0 += 16) {
    const SeqChunk c = SeqLoad(w, k0, n);
#pragma unroll
    for (int j = 0; j < 16; ++j) sum += c.v[j];
  }
  return sum;
}
// Entry j of a chunk's 16 values (a select chain, not a dynamic register index).
__device__ __forceinline__ double SeqPick(const double (&c)[16], std::uint32_t j) {
  double v = c[0];
#pragma unroll
  for (std::uint32_t i = 1; i < 16; ++i) v = i == j ? c[i] : v;
  return v;
}
// The first k (1-based) with k >= minimum and w[0] + ... + w[k-1] >= target, scanning at most n entries; n + 1
// when the scan ends first. The weights are >= 0, so the rounded running sum never decreases: a chunk holds the
// first crossing exactly when its last sum crosses, so only that sum is tested per chunk (the chain costs one add
// per element) and the crossing chunk's sums are searched once. *at_cut receives w[0] + ... + w[k-1] when k is the
// crossing itself (the same adds in the same order as SeqSum over k entries), else -1.
__device__ std::uint32_t SeqCut(const double* w, std::uint32_t n, std::uint32_t minimum, double target,
                                double* at_cut) {
  *at_cut = -1.0;
  double cum = 0.0;
  for (std::uint32_t k0 = 0; k0 < n; k0 += 16) {
    const SeqChunk c = SeqLoad(w, k0, n);
    double cs[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      cum += c.v[j];
      cs[j] = cum;
    }
    if (cum >= target) {  // entries past n add +0.0, so the crossing lies below n
      std::uint32_t hit = 0;
#pragma unroll
      for (int j = 0; j < 16; ++j) hit |= static_cast<std::uint32_t>(cs[j] >= target) << j;
      const std::uint32_t j = __builtin_ctz(hit), k = k0 + j + 1;
      if (k >= minimum) {
        *at_cut = SeqPick(cs, j);
        return k;
      }
      return minimum <= n ? minimum : n + 1;  // the sums only grow: the first k >= minimum crosses too
    }
  }
  return n + 1;
}
// The first i with u - p[0] - ... - p[i] < 0, or n when none (the remainder never grows: p >= 0).
__device__ std::uint32_t SeqWalk(const double* pr, std::uint32_t n, double u) {
  double r = u;
  for (std::uint32_t k0 = 0; k0 < n; k0 += 16) {
    const SeqChunk c = SeqLoad(pr, k0, n);
    double rs[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      r -= c.v[j];
      rs[j] = r;
    }
    if (r < 0.0) {
      std::uint32_t hit = 0;
#pragma unroll
      for (int j = 0; j < 16; ++j) hit |= static_cast<std::uint32_t>(rs[j] < 0.0) << j;
      return k0 + __builtin_ctz(hit);
    }
  }
  return n;
}

// The histogram cut of the sorted path: the bins [0, cut] hold the candidates sorted on chip. Rc = min(K0, cap)
// candidates are needed; the bin where the count reaches Rc is the cut when the bins up to it fit the cap. When they
// do not, a top-k row (which needs all of its K0) falls back to an exact radix selection (returns false); a row
// without top-k takes the bins before it (still a full prefix of the sorted order), unless that is empty.
__device__ bool HistCut(const std::uint32_t* hist, std::uint32_t Rc, bool topk, std::uint32_t* cut,
                        std::uint32_t* red, std::uint32_t* out2) {
  constexpr std::uint32_t per = kBins / kThreads;  // both callers run kThreads threads
  std::uint32_t h[per], c = 0;
#pragma unroll
  for (std::uint32_t j = 0; j < per; ++j) {
    h[j] = hist[threadIdx.x * per + j];  // read once, kept for the crossing search
    c += h[j];
  }
  std::uint32_t tot;
  std::uint32_t base = BlockExclScan(c, red, &tot);
  if (threadIdx.x == 0) {
    out2[0] = 0xFFFFFFFFu;
    out2[1] = 0;
  }
  __syncthreads();
#pragma unroll
  for (std::uint32_t j = 0; j < per; ++j) {
    const std::uint32_t bin = threadIdx.x * per + j;
    if (base < Rc && base + h[j] >= Rc) {
      out2[0] = bin;
      out2[1] = base;  // count before the crossing bin
      out2[2] = base + h[j];
    }
    base += h[j];
  }
  __syncthreads();
  const std::uint32_t bc = out2[0], before = out2[1], through = out2[2];
  __syncthreads();
  if (bc == 0xFFFFFFFFu) return false;
  if (through <= kCap) {
    *cut = bc;
    return true;
  }
  if (topk || before == 0) return false;
  *cut = bc - 1;
  return true;
}

}  // namespace halo::sample

// ---- pass 1: penalized values and per-block maxima ---------------------------------------------------------------
// grid (nb, rows), block 1024; slice b of row r: tokens [4096 b, 4096 b + 4096). Also clears the row's histogram
// and candidate counter for the later passes.
extern "C" __global__ void __launch_bounds__(1024)
    halo_sample_prep(const float* __restrict__ logits, std::uint64_t row_stride,
                     const HaloSampleParams* __restrict__ params, const HaloPenalty* __restrict__ penalties,
                     std::uint32_t pen_stride, std::uint32_t V, std::uint32_t rows, void* ws) {
  using namespace halo::sample;
  __shared__ std::uint32_t bm[kSampleSlice / 32];
  __shared__ std::uint32_t prange[2];
  __shared__ unsigned long long rk[kWaves];
  __shared__ std::uint32_t rt[kWaves], ru[kWaves];
  const std::uint32_t row = blockIdx.y, b = blockIdx.x, t = threadIdx.x, nb = gridDim.x;
  const HaloSampleParams p = params[row];
  if (BadParams(p, V, pen_stride)) return;
  const Ws w = Carve(ws, rows, V);
  for (std::uint32_t i = b * blockDim.x + t; i < kBins; i += nb * blockDim.x)
    w.hist[static_cast<std::size_t>(row) * kBins + i] = 0;
  if (b == 0 && t == 0) w.cn[row] = 0;
  const float* x = logits + row * row_stride;
  const HaloPenalty* pen = penalties + static_cast<std::size_t>(row) * pen_stride;
  const std::uint32_t lo = b * kSampleSlice, hi = min(V, lo + kSampleSlice);
  const std::uint32_t npen = p.n_penalties;
  if (npen) {
    for (std::uint32_t i = t; i < kSampleSlice / 32; i += blockDim.x) bm[i] = 0;
    if (t < 2) {  // first entry with token >= lo (t = 0) / >= hi (t = 1)
      const std::uint32_t key = t == 0 ? lo : hi;
      std::uint32_t a = 0, z = npen;
      while (a < z) {
        const std::uint32_t mid = (a + z) / 2;
        if (pen[mid].token < key) a = mid + 1;
        else z = mid;
      }
      prange[t] = a;
    }
    __syncthreads();
    for (std::uint32_t j = prange[0] + t; j < prange[1]; j += blockDim.x) {
      const std::uint32_t tk = pen[j].token;
      if (tk >= lo && tk < hi) atomicOr(&bm[(tk - lo) >> 5], 1u << ((tk - lo) & 31));
    }
    __syncthreads();
  }
  std::uint64_t best_k = kNoBound;
  std::uint32_t best_t = 0xFFFFFFFFu, nf = 0;
  double* val = w.val + static_cast<std::size_t>(row) * V;
  constexpr int kPer = kSampleSlice / kThreads;
  float lv[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const std::uint32_t i = lo + t + kThreads * j;
    lv[j] = i < hi ? x[i] : -INFINITY;
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const std::uint32_t i = lo + t + kThreads * j;
    if (i >= hi) continue;
    double a = -INFINITY;
    if (isfinite(lv[j])) {
      a = lv[j];
      if (npen && (bm[(i - lo) >> 5] >> ((i - lo) & 31)) & 1u) {
        std::uint32_t q = prange[0], z = prange[1];
        while (q < z) {
          const std::uint32_t mid = (q + z) / 2;
          if (pen[mid].token < i) q = mid + 1;
          else z = mid;
        }
        if (q < prange[1] && pen[q].token == i) a = Penalize(a, p, pen[q]);
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
  // only thread 0 needs the block's results: wave reductions, one barrier, thread 0 combines the waves in
  // BlockSum / BlockMinPair order
  nf = WaveSum(nf);
  WaveMinPair(best_k, best_t);
  if (t % kWave == 0) {
    ru[t / kWave] = nf;
    rk[t / kWave] = best_k;
    rt[t / kWave] = best_t;
  }
  __syncthreads();
  if (t == 0) {
    std::uint32_t n = 0, tk = rt[0];
    std::uint64_t k = rk[0];
    for (std::uint32_t i = 0; i < kWaves; ++i) {
      n += ru[i];
      if (rk[i] < k || (rk[i] == k && rt[i] < tk)) {
        k = rk[i];
        tk = rt[i];
      }
    }
    const std::size_t o = static_cast<std::size_t>(row) * nb + b;
    w.pkey[o] = k;
    w.ptok[o] = tk;
    w.pnf[o] = n;
  }
}

// ---- pass 2: weights (linear path) or the histogram and full weight sum (sorted path) ----------------------------
// grid (nb, rows), block 1024.
extern "C" __global__ void __launch_bounds__(1024)
    halo_sample_weights(const HaloSampleParams* __restrict__ params, std::uint32_t pen_stride, std::uint32_t V,
                        std::uint32_t rows, void* ws) {
  using namespace halo::sample;
  __shared__ double rd[kWaves];
  __shared__ std::uint32_t ru[kWaves];
  __shared__ unsigned long long rk[kWaves], rm[kWaves];
  __shared__ std::uint32_t rt[kWaves];
  __shared__ std::uint32_t lh[kBins];
  const std::uint32_t row = blockIdx.y, b = blockIdx.x, t = threadIdx.x, nb = gridDim.x;
  const HaloSampleParams p = params[row];
  if (BadParams(p, V, pen_stride)) return;
  const Ws w = Carve(ws, rows, V);
  const RowMax m = ReduceParts(w, row, nb, rk, rt, ru);
  if (m.nf == 0 || p.temperature == 0.0f) return;
  const double M = KeyValue(m.key), T = p.temperature;
  double* val = w.val + static_cast<std::size_t>(row) * V;
  const std::uint32_t lo = b * kSampleSlice, hi = min(V, lo + kSampleSlice);
  constexpr int kPer = kSampleSlice / kThreads;
  const std::size_t o = static_cast<std::size_t>(row) * nb + b;
  if (LinearPath(p)) {
    const double thr = p.min_p > 0.0f ? M + T * log(static_cast<double>(p.min_p)) : -INFINITY;
    double sum = 0.0, minw = INFINITY;
    std::uint32_t nz = 0, last = 0;
    double av[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const std::uint32_t i = lo + t + kThreads * j;
      av[j] = i < hi ? val[i] : -INFINITY;
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const std::uint32_t i = lo + t + kThreads * j;
      if (i >= hi) continue;
      const double a = av[j];
      const double wt = (a != -INFINITY && a >= thr) ? exp((a - M) / T) : 0.0;
      val[i] = wt;
      sum += wt;
      if (wt != 0.0) {
        ++nz;
        last = i + 1;
        minw = fmin(minw, wt);
      }
    }
    // only thread 0 needs the block's results: wave reductions, one barrier, thread 0 adds the wave sums in
    // BlockSum order (the minima are order-free)
    sum = WaveSum(sum);
    nz = WaveSum(nz);
    std::uint64_t lk = ~static_cast<std::uint64_t>(last);
    std::uint32_t lt = 0;
    WaveMinPair(lk, lt);
    std::uint64_t mk = static_cast<std::uint64_t>(__double_as_longlong(minw));  // positive doubles order as bits
    std::uint32_t mt = 0;
    WaveMinPair(mk, mt);
    if (t % kWave == 0) {
      rd[t / kWave] = sum;
      ru[t / kWave] = nz;
      rk[t / kWave] = lk;
      rm[t / kWave] = mk;
    }
    __syncthreads();
    if (t == 0) {
      double s0 = 0.0;
      std::uint32_t z = 0;
      std::uint64_t l = rk[0], m = rm[0];
      for (std::uint32_t i = 0; i < kWaves; ++i) {
        s0 += rd[i];
        z += ru[i];
        l = min(l, static_cast<std::uint64_t>(rk[i]));
        m = min(m, static_cast<std::uint64_t>(rm[i]));
      }
      w.psum[o] = s0;
      w.pnz[o] = z;
      w.plast[o] = static_cast<std::uint32_t>(~l);
      w.pminw[o] = __longlong_as_double(static_cast<long long>(m));
    }
    return;
  }
  const bool has_full = p.top_k == 0 && p.top_p < 1.0f && V > 1024;
  for (std::uint32_t i = t; i < kBins; i += blockDim.x) lh[i] = 0;
  __syncthreads();
  double sum = 0.0;
  double av[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const std::uint32_t i = lo + t + kThreads * j;
    av[j] = i < hi ? val[i] : -INFINITY;
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const double a = av[j];
    if (a == -INFINITY) continue;
    if (has_full) sum += exp((a - M) / T);
    atomicAdd(&lh[Bin(M, a)], 1u);
  }
  __syncthreads();
  for (std::uint32_t i = t; i < kBins; i += blockDim.x)
    if (lh[i]) atomicAdd(&w.hist[static_cast<std::size_t>(row) * kBins + i], lh[i]);
  sum = BlockSum(sum, rd);
  if (t == 0) w.psum[o] = sum;
}

// ---- pass 3: candidates of the sorted path -----------------------------------------------------------------------
// grid (nb, rows), block 1024: every block finds the same histogram cut and appends its tokens in the bins up to it.
extern "C" __global__ void __launch_bounds__(1024)
    halo_sample_collect(const HaloSampleParams* __restrict__ params, std::uint32_t pen_stride, std::uint32_t V,
                        std::uint32_t rows, void* ws) {
  using namespace halo::sample;
  __shared__ unsigned long long rk[kWaves];
  __shared__ std::uint32_t rt[kWaves], ru[kWaves], o2[3], count, base;
  const std::uint32_t row = blockIdx.y, b = blockIdx.x, t = threadIdx.x, nb = gridDim.x;
  const HaloSampleParams p = params[row];
  if (BadParams(p, V, pen_stride)) return;
  const Ws w = Carve(ws, rows, V);
  const RowMax m = ReduceParts(w, row, nb, rk, rt, ru);
  if (m.nf == 0 || p.temperature == 0.0f || LinearPath(p)) return;
  const std::uint32_t floor_keep = p.min_keep > 1 ? p.min_keep : 1;
  const std::uint64_t keep_cfg =
      p.top_k > 0 ? min(static_cast<std::uint64_t>(V), static_cast<std::uint64_t>(max(p.top_k, floor_keep)))
                  : static_cast<std::uint64_t>(V);
  const std::uint32_t K0 = static_cast<std::uint32_t>(min(static_cast<std::uint64_t>(m.nf), keep_cfg));
  std::uint32_t cut;
  if (!HistCut(w.hist + static_cast<std::size_t>(row) * kBins, min(K0, kCap), p.top_k > 0, &cut, ru, o2)) return;
  const double M = KeyValue(m.key);
  const double* val = w.val + static_cast<std::size_t>(row) * V;
  const std::uint32_t lo = b * kSampleSlice, hi = min(V, lo + kSampleSlice);
  constexpr int kPer = kSampleSlice / kThreads;
  if (t == 0) count = 0;
  __syncthreads();
  std::uint32_t slot[kPer];
  double av[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const std::uint32_t i = lo + t + kThreads * j;
    av[j] = i < hi ? val[i] : -INFINITY;
    slot[j] = av[j] != -INFINITY && Bin(M, av[j]) <= cut ? atomicAdd(&count, 1u) : 0xFFFFFFFFu;
  }
  __syncthreads();
  if (t == 0) base = count ? atomicAdd(&w.cn[row], count) : 0;  // one reservation per block
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kPer; ++j)
    if (slot[j] != 0xFFFFFFFFu) {
      const std::size_t o = static_cast<std::size_t>(row) * kCap + base + slot[j];
      w.ckey[o] = DescKey(av[j]);
      w.ctok[o] = lo + t + kThreads * j;
    }
}

// ---- pass 4: the draw --------------------------------------------------------------------------------------------
// grid rows, block 1024. logits are read only through pass 1; out [rows].
extern "C" __global__ void __launch_bounds__(1024)
    halo_sample_final(const HaloSampleParams* __restrict__ params, std::uint32_t pen_stride, std::uint32_t V,
                      std::uint32_t rows, void* ws, HaloSampleOut* __restrict__ outs) {
  using namespace halo::sample;
  __shared__ Lds s;
  const std::uint32_t row = blockIdx.x, t = threadIdx.x, nb = Blocks(V);
  const HaloSampleParams p = params[row];
  HaloSampleOut* out = outs + row;
  std::uint64_t rng = p.rng;
  if (BadParams(p, V, pen_stride)) {
    Finish(out, HALO_SAMPLE_BAD_PARAMS, 0, rng);
    return;
  }
  const Ws w = Carve(ws, rows, V);
  const RowMax m = ReduceParts(w, row, nb, s.rq, s.ru + 0, s.ru);
  const std::uint64_t best_k = m.key;
  const std::uint32_t best_t = m.tok, nf = m.nf;
  if (nf == 0) {
    Finish(out, HALO_SAMPLE_NO_FINITE, 0, rng);
    return;
  }
  if (p.temperature == 0.0f) {
    Finish(out, best_t, 1, rng);
    return;
  }
  double* val = w.val + static_cast<std::size_t>(row) * V;
  unsigned long long* fx = w.fx + static_cast<std::size_t>(row) * V;
  const std::size_t po = static_cast<std::size_t>(row) * nb;
  const double M = KeyValue(best_k);
  const double T = p.temperature;
  const std::uint32_t floor_keep = p.min_keep > 1 ? p.min_keep : 1;

  // linear path: token order; val holds the weights
  if (LinearPath(p)) {
    // per-slice partials, one per thread (nb <= 64)
    double ps = 0.0, mw = INFINITY;
    std::uint32_t pz = 0, pl = 0;
    if (t < nb) {
      ps = w.psum[po + t];
      pz = w.pnz[po + t];
      pl = w.plast[po + t];
      if (pz) mw = w.pminw[po + t];
    }
    // wave 0 holds them all: its shuffle trees give the block reductions' results, one broadcast
    if (t < kWave) {  // ps stays this thread's slice sum (the slice search below reads it)
      const double sum = WaveSum(ps);
      const std::uint32_t nz = WaveSum(pz);
      std::uint64_t lk = ~static_cast<std::uint64_t>(pl);
      std::uint32_t lt = 0;
      WaveMinPair(lk, lt);
      std::uint64_t mk = static_cast<std::uint64_t>(__double_as_longlong(mw));  // positive doubles order as bits
      std::uint32_t mt = 0;
      WaveMinPair(mk, mt);
      if (t == 0) {
        s.xd = sum;
        s.xu = nz;
        s.xq[0] = lk;
        s.xq[1] = mk;
      }
    }
    __syncthreads();
    const double total = s.xd;
    std::uint32_t live = s.xu;
    std::uint32_t last = static_cast<std::uint32_t>(~s.xq[0]);
    const std::uint64_t mk = s.xq[1];
    const bool exact_count = __longlong_as_double(static_cast<long long>(mk)) / total != 0.0;
    if (!exact_count) {  // weights near the underflow of w / total: count the way the CPU drops them
      std::uint32_t nz = 0, lst = 0;
      for (std::uint32_t i = t; i < V; i += kThreads)
        if (val[i] / total != 0.0) {
          ++nz;
          lst = i + 1;
        }
      live = BlockSumU(nz, s);
      std::uint64_t lk2 = ~static_cast<std::uint64_t>(lst);
      std::uint32_t lt2 = 0;
      BlockMinPair(lk2, lt2, s);
      last = static_cast<std::uint32_t>(~lk2);
    }
    const std::uint32_t last_nz = last - 1;
    if (live == 1) {
      Finish(out, last_nz, 1, rng);
      return;
    }
    const double u = Uniform(&rng);
    // the slice whose weights hold the uniform (a scan of the slice masses), then the 4-token range within it
    const double pb = t < nb ? ps / total : 0.0;
    double ptot;
    const double acc = BlockExclScan(pb, s.rd, &ptot);
    if (t == 0) {
      s.bu[3] = 0xFFFFFFFFu;
      s.bu[1] = 0xFFFFFFFFu;
    }
    __syncthreads();
    if (t < nb && pb > 0.0 && u - acc < pb) atomicMin(&s.bu[3], t);
    __syncthreads();
    if (t == s.bu[3]) s.bd[1] = acc;
    __syncthreads();
    const std::uint32_t hit = s.bu[3];
    if (hit != 0xFFFFFFFFu) {
      const double r0 = u - s.bd[1];
      const std::uint32_t lo = min(V, hit * kSampleSlice + t * 4), hi = min(V, lo + 4);
      double ps = 0.0;
      for (std::uint32_t i = lo; i < hi; ++i) ps += val[i] / total;
      double tot;
      const double ex = BlockExclScan(ps, s.rd, &tot);
      if (ps > 0.0 && r0 >= ex && r0 < ex + ps) {
        double r = r0 - ex;
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
    }
    __syncthreads();
    const std::uint32_t pick = s.bu[1];
    Finish(out, pick == 0xFFFFFFFFu ? last_nz : pick, live, rng);
    return;
  }

  // sorted path: the candidates of pass 3, or an exact radix selection of the best Rc
  const std::uint64_t keep_cfg =
      p.top_k > 0 ? min(static_cast<std::uint64_t>(V), static_cast<std::uint64_t>(max(p.top_k, floor_keep)))
                  : static_cast<std::uint64_t>(V);
  const std::uint32_t K0 = static_cast<std::uint32_t>(min(static_cast<std::uint64_t>(nf), keep_cfg));
  std::uint32_t Rc = min(K0, kCap);
  const bool has_full = p.top_k == 0 && p.top_p < 1.0f && V > 1024;
  double full_sum = 0.0;
  if (has_full) full_sum = BlockSumD(t < nb ? w.psum[po + t] : 0.0, s);
  std::uint32_t cut;
  const bool collected =
      HistCut(w.hist + static_cast<std::size_t>(row) * kBins, Rc, p.top_k > 0, &cut, s.ru, s.bu + 4);
  std::uint32_t n;
  bool sorted = false;
  if (collected) {
    // The candidates are every token in bins 0..cut: values within (cut + 1) / 64 of the maximum. They are counted
    // again on chip over kBins finer bins spanning that range (the coarse bins themselves when the last one, which is
    // open-ended, is in), a scan of the counts gives each bin's place in the sorted list, and the candidates are
    // scattered to their bin's range and ranked within it (a few per bin, so the rank loop is short), unless a bin
    // is too full for that. The bin is a non-decreasing function of max - value, so bin order is list order.
    n = w.cn[row];
    constexpr std::uint32_t kPerE = kCap / kThreads;  // n <= kCap
    constexpr std::uint32_t kPerT = kBins / kThreads;
    std::uint64_t gk[kPerE];
    std::uint32_t gt[kPerE], gb[kPerE];
#pragma unroll
    for (std::uint32_t j = 0; j < kPerE; ++j) {
      const std::uint32_t i = t + kThreads * j;
      if (i < n) {
        gk[j] = w.ckey[static_cast<std::size_t>(row) * kCap + i];
        gt[j] = w.ctok[static_cast<std::size_t>(row) * kCap + i];
      }
    }
    // (max - value) * 64 is exact, so scale 64 reproduces the coarse bins
    const double scale = cut < kBins - 1 ? static_cast<double>(kBins) * 64.0 / static_cast<double>(cut + 1) : 64.0;
    const auto bin_of = [&](std::uint64_t k) -> std::uint32_t {
      const double d = (M - KeyValue(k)) * scale;
      return d < static_cast<double>(kBins) ? static_cast<std::uint32_t>(d) : kBins - 1;
    };
#pragma unroll
    for (std::uint32_t j = 0; j < kPerT; ++j) s.b.hist[t * kPerT + j] = 0;
    if (t == 0) s.bu[7] = 0;
    __syncthreads();
    // the largest bin count is the largest count any increment returns: a wave maximum, one LDS maximum
    std::uint32_t cm = 0;
#pragma unroll
    for (std::uint32_t j = 0; j < kPerE; ++j)
      if (t + kThreads * j < n) {
        gb[j] = bin_of(gk[j]);
        cm = max(cm, atomicAdd(&s.b.hist[gb[j]], 1u) + 1);
      }
    for (int o = kWave / 2; o > 0; o >>= 1) cm = max(cm, static_cast<std::uint32_t>(__shfl_xor(cm, o, kWave)));
    if (t % kWave == 0 && cm) atomicMax(&s.bu[7], cm);
    __syncthreads();
    const std::uint32_t cmax = s.bu[7];
    std::uint32_t c[kPerT], c4 = 0;
#pragma unroll
    for (std::uint32_t j = 0; j < kPerT; ++j) {
      c[j] = s.b.hist[t * kPerT + j];
      c4 += c[j];
    }
    std::uint32_t tot;
    std::uint32_t start = BlockExclScan(c4, s.ru, &tot);  // its barriers order the reads above before the writes
#pragma unroll
    for (std::uint32_t j = 0; j < kPerT; ++j) {
      s.b.hist[t * kPerT + j] = start;  // bin start
      s.a.bitmap[t * kPerT + j] = 0;    // bin fill counter
      start += c[j];
    }
    __syncthreads();  // starts and cleared counters before any scatter
    if (cmax <= 512) {
#pragma unroll
      for (std::uint32_t j = 0; j < kPerE; ++j)
        if (t + kThreads * j < n) {
          const std::uint32_t at = s.b.hist[gb[j]] + atomicAdd(&s.a.bitmap[gb[j]], 1u);
          s.key[at] = gk[j];
          s.tok[at] = gt[j];
        }
      __syncthreads();
      // rank within the bin by (key, token), then move every element to start + rank
      std::uint64_t ek[kPerE];
      std::uint32_t et[kPerE], pos[kPerE];
#pragma unroll
      for (std::uint32_t j = 0; j < kPerE; ++j) {
        const std::uint32_t i = t + kThreads * j;
        pos[j] = 0xFFFFFFFFu;
        if (i < n) {
          ek[j] = s.key[i];
          et[j] = s.tok[i];
          const std::uint32_t bin = bin_of(ek[j]);
          const std::uint32_t b0 = s.b.hist[bin], cnt = s.a.bitmap[bin];
          std::uint32_t r = 0;
          for (std::uint32_t q0 = b0; q0 < b0 + cnt; q0 += 4) {  // four reads in flight per step
            std::uint64_t kq[4];
            std::uint32_t tq[4];
#pragma unroll
            for (std::uint32_t u = 0; u < 4; ++u) {
              const std::uint32_t q = min(q0 + u, kCap - 1);
              kq[u] = s.key[q];
              tq[u] = s.tok[q];
            }
#pragma unroll
            for (std::uint32_t u = 0; u < 4; ++u)  // bitwise, not short-circuit: no branches
              r += static_cast<std::uint32_t>((q0 + u < b0 + cnt) &
                                              ((kq[u] < ek[j]) | ((kq[u] == ek[j]) & (tq[u] < et[j]))));
          }
          pos[j] = b0 + r;
        }
      }
      __syncthreads();
#pragma unroll
      for (std::uint32_t j = 0; j < kPerE; ++j)
        if (pos[j] != 0xFFFFFFFFu) {
          s.key[pos[j]] = ek[j];
          s.tok[pos[j]] = et[j];
        }
      sorted = true;
    } else {
#pragma unroll
      for (std::uint32_t j = 0; j < kPerE; ++j)
        if (t + kThreads * j < n) {
          s.key[t + kThreads * j] = gk[j];
          s.tok[t + kThreads * j] = gt[j];
        }
    }
    Rc = min(n, K0);
  } else {
    std::uint64_t ck;
    std::uint32_t ct;
    unsigned long long bn, bm;
    Select(val, nullptr, V, Rc, kNoBound, 0xFFFFFFFFu, s, &ck, &ct, &bn, &bm);
    if (t == 0) s.bu[4] = 0;
    __syncthreads();
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
    __syncthreads();
    n = s.bu[4];
  }
  __syncthreads();
  std::uint32_t P = 1;
  while (!sorted && P < n) P <<= 1;
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
  // 4. top-p, min-p and the weight sum in list order (the CPU's order; the sums on one lane)
  const std::uint32_t minimum = min(K0, floor_keep);
  if (t == 0) {
    std::uint32_t keep = K0;
    bool large = false;
    double cut_sum = -1.0;  // the sum over the kept prefix when the top-p cut produced it
    if (p.top_p < 1.0f && K0 > 1) {
      double sum = full_sum;
      if (!has_full) {
        if (K0 > Rc) large = true;
        else sum = SeqSum(s.a.w, K0);
      }
      if (!large) {
        double at_cut;
        const std::uint32_t k =
            SeqCut(s.a.w, min(K0, Rc), minimum, static_cast<double>(p.top_p) * sum, &at_cut);
        if (k > min(K0, Rc)) {
          if (Rc < K0) large = true;  // the cut lies past the sorted candidates
          else keep = K0;
        } else {
          keep = k;
          cut_sum = at_cut;
        }
      }
    }
    s.bu[5] = keep;
    s.bu[6] = large;
    s.bd[2] = cut_sum;
  }
  __syncthreads();
  const std::uint32_t keep_top_p = s.bu[5];
  const double cut_sum = s.bd[2];
  std::uint32_t keep = keep_top_p;
  bool large = s.bu[6] != 0;
  __syncthreads();
  if (!large && p.min_p > 0.0f && keep > 1) {
    // the candidates are sorted, so those at or above the threshold are a prefix: count them
    const double thr = M + T * log(static_cast<double>(p.min_p));
    const std::uint32_t lim = min(keep, Rc);
    std::uint32_t c = 0;
    for (std::uint32_t i = t; i < lim; i += kThreads) c += KeyValue(s.key[i]) >= thr;
    c = BlockSumU(c, s);
    if (c == Rc && Rc < keep) large = true;
    else keep = min(keep, max(c, minimum));
  }
  if (!large && keep > Rc) large = true;
  if (!large) {
    // the cut's own running sum when min-p kept the whole top-p prefix (bitwise SeqSum over it)
    if (t == 0) s.bd[0] = keep == keep_top_p && cut_sum >= 0.0 ? cut_sum : SeqSum(s.a.w, keep);
    __syncthreads();
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
    // only thread 0 draws: wave reductions, one barrier, thread 0 combines the waves
    nz = WaveSum(nz);
    std::uint64_t lk = ~static_cast<std::uint64_t>(last);
    std::uint32_t lt = 0;
    WaveMinPair(lk, lt);
    if (t % kWave == 0) {
      s.ru[t / kWave] = nz;
      s.rq[t / kWave] = lk;
    }
    __syncthreads();
    if (t == 0) {
      std::uint32_t live = 0;
      std::uint64_t l = s.rq[0];
      for (std::uint32_t i = 0; i < kWaves; ++i) {
        live += s.ru[i];
        l = min(l, static_cast<std::uint64_t>(s.rq[i]));
      }
      const std::uint32_t last_nz = static_cast<std::uint32_t>(~l) - 1;
      std::uint32_t token = s.tok[last_nz];
      if (live > 1) {
        const std::uint32_t i = SeqWalk(s.a.w, keep, Uniform(&rng));
        if (i < keep) token = s.tok[i];
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
  keep = K0;
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
