// GQA decode attention over a paged KV cache shared by a ragged batch of sessions (gfx950, wave64).
//
// Reference semantics: ReferenceModel::Attention dense branch (src/model/reference.cpp:368-416, 492-527) and the
// GPU halo_attention_decode / halo_attention_select_b (src/kernels/core.hip:514-544, 898): per query head h (kv
// head h / G), o = softmax(q . K^T / sqrt(d)) V, then o *= sigmoid(gate).
//
// KV layout in HBM: pages of 16 tokens; K and V pools [page][kv_head][16][d] fp32; each session has a page table
// [max_pages]. Sessions of one batch share their first `prefix` tokens (identical page-table entries): a prefix
// chunk is read once and scored against the queries of every session (S * G query vectors), a suffix chunk only
// against its own session's G queries. Each (kv head, 32-token chunk) is one block producing flash partials
// (running max, sum, weighted V); halo_attn_decode_combine merges them per (session, head) and applies the gate.
#include "common.h"

using halo::kWave;

namespace {
constexpr int kHd = 256;      // head dim
constexpr int kPage = 16;     // tokens per page
constexpr int kChunk = 32;    // tokens per block
constexpr int kMaxQ = 32;     // query vectors per block (sessions * G)
}  // namespace

// grid (Hkv * (prefix_chunks + S * suffix_chunks)), block 256.
//   q [S][Hq][256]; kpool, vpool [pages][Hkv][16][256]; pages [S][max_pages]; nkv [S] visible positions;
//   partial m, l [items][S * G], acc [items][S * G][256] (item = blockIdx.x).
// Prefix chunks cover tokens [32 c, 32 c + 32) < prefix of every session; suffix chunk c of session s covers
// [prefix + 32 c, ...) up to nkv[s]; positions at or past nkv[s] are masked, empty chunks record m = -inf.
extern "C" __global__ void __launch_bounds__(256) halo_attn_decode_partial(
    const float* __restrict__ q, const float* __restrict__ kpool, const float* __restrict__ vpool,
    const std::uint32_t* __restrict__ pages, const std::uint32_t* __restrict__ nkv, float* __restrict__ pm,
    float* __restrict__ pl, float* __restrict__ pacc, std::uint32_t S, std::uint32_t Hq, std::uint32_t Hkv,
    std::uint32_t prefix, std::uint32_t max_pages, std::uint32_t prefix_chunks, std::uint32_t suffix_chunks) {
  __shared__ float qs[kMaxQ][kHd];       // 32 KB
  __shared__ float ps[kMaxQ][kChunk + 1];
  static_assert(kChunk <= kWave, "a chunk's tokens are the lanes of a wave");
  const std::uint32_t G = Hq / Hkv, x = blockIdx.x, kvh = x % Hkv, c = x / Hkv;
  const std::uint32_t t = threadIdx.x, wave = t / kWave, lane = t % kWave;
  const bool is_prefix = c < prefix_chunks;
  const std::uint32_t sess = is_prefix ? 0 : (c - prefix_chunks) / suffix_chunks;
  const std::uint32_t start = is_prefix ? c * kChunk : prefix + ((c - prefix_chunks) % suffix_chunks) * kChunk;
  const std::uint32_t nq = is_prefix ? S * G : G;
  const std::uint32_t limit = is_prefix ? prefix : nkv[sess];
  const std::uint32_t slots = S * G;
  float* m_out = pm + static_cast<std::size_t>(x) * slots;
  float* l_out = pl + static_cast<std::size_t>(x) * slots;
  float* a_out = pacc + static_cast<std::size_t>(x) * slots * kHd;
  if (start >= limit) {
    if (t < nq) {
      const std::uint32_t slot = is_prefix ? t : sess * G + t;
      m_out[slot] = -INFINITY;
      l_out[slot] = 0.0f;
    }
    return;
  }
  // queries of this kv head: slot i = session * G + g (prefix) or g (suffix)
  for (std::uint32_t i = t; i < nq * (kHd / 4); i += blockDim.x) {
    const std::uint32_t qi = i / (kHd / 4), d4 = i % (kHd / 4);
    const std::uint32_t s = is_prefix ? qi / G : sess, g = is_prefix ? qi % G : qi;
    const float4 v = reinterpret_cast<const float4*>(q + (static_cast<std::size_t>(s) * Hq + kvh * G + g) * kHd)[d4];
    reinterpret_cast<float4*>(&qs[qi][0])[d4] = v;
  }
  __syncthreads();
  // scores: lane = token of the chunk, wave = a quarter of the queries
  const std::uint32_t tok = start + lane;
  const bool live = lane < static_cast<std::uint32_t>(kChunk) && tok < limit;
  const std::uint32_t page = pages[static_cast<std::size_t>(sess) * max_pages + min(tok, limit - 1) / kPage];
  const float* krow = kpool + ((static_cast<std::size_t>(page) * Hkv + kvh) * kPage + (tok % kPage)) * kHd;
  const float scale = 1.0f / sqrtf(static_cast<float>(kHd));
  const std::uint32_t per_wave = (nq + 3) / 4;
  constexpr int kQPerWave = kMaxQ / 4;
  float sc[kQPerWave];
#pragma unroll
  for (int i = 0; i < kQPerWave; ++i) sc[i] = 0.0f;
  constexpr int kKU = 16;  // row pieces loaded ahead of their arithmetic
  for (std::uint32_t d0 = 0; d0 < kHd / 4; d0 += kKU) {
    float4 kv[kKU];
#pragma unroll
    for (int u = 0; u < kKU; ++u) kv[u] = reinterpret_cast<const float4*>(krow)[d0 + u];
#pragma unroll
    for (int u = 0; u < kKU; ++u)
#pragma unroll
      for (int i = 0; i < kQPerWave; ++i) {
        const std::uint32_t qi = wave * per_wave + i;
        if (i < static_cast<int>(per_wave) && qi < nq) {
          const float4 qv = reinterpret_cast<const float4*>(&qs[qi][0])[d0 + u];
          sc[i] += kv[u].x * qv.x + kv[u].y * qv.y + kv[u].z * qv.z + kv[u].w * qv.w;
        }
      }
  }
#pragma unroll
  for (int i = 0; i < kQPerWave; ++i) {
    const std::uint32_t qi = wave * per_wave + i;
    if (i < static_cast<int>(per_wave) && qi < nq) {
      const float s = live ? sc[i] * scale : -INFINITY;
      const float m = halo::GroupMax(s);
      const float p = live ? expf(s - m) : 0.0f;
      const float l = halo::GroupSum(p);
      if (lane < static_cast<std::uint32_t>(kChunk)) ps[qi][lane] = p;
      if (lane == 0) {
        const std::uint32_t slot = is_prefix ? qi : sess * G + qi;
        m_out[slot] = m;
        l_out[slot] = l;
      }
    }
  }
  __syncthreads();
  // weighted V: thread = one of the 256 dims, all queries; the chunk's page ids are read once
  float acc[kMaxQ];
#pragma unroll
  for (int i = 0; i < kMaxQ; ++i) acc[i] = 0.0f;
  const std::uint32_t ntok = min(static_cast<std::uint32_t>(kChunk), limit - start);
  std::uint32_t pgs[kChunk / kPage];
#pragma unroll
  for (int i = 0; i < kChunk / kPage; ++i)
    pgs[i] = pages[static_cast<std::size_t>(sess) * max_pages + min(start / kPage + i, (limit - 1) / kPage)];
  constexpr int kU = 8;
  for (std::uint32_t j0 = 0; j0 < ntok; j0 += kU) {
    float vv[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const std::uint32_t j = min(j0 + u, ntok - 1);
      const std::uint32_t pg = pgs[j / kPage];
      vv[u] = vpool[((static_cast<std::size_t>(pg) * Hkv + kvh) * kPage + ((start + j) % kPage)) * kHd + t];
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (j0 + u >= ntok) break;
#pragma unroll
      for (int i = 0; i < kMaxQ; ++i)
        if (i < static_cast<int>(nq)) acc[i] += ps[i][j0 + u] * vv[u];
    }
  }
#pragma unroll
  for (int i = 0; i < kMaxQ; ++i)
    if (i < static_cast<int>(nq)) {
      const std::uint32_t slot = is_prefix ? i : sess * G + i;
      a_out[static_cast<std::size_t>(slot) * kHd + t] = acc[i];
    }
}

// grid (S * Hq), block 256: merges the partials of session s, head h over its prefix and suffix chunks
// (log-sum-exp), o = acc / l, then o *= sigmoid(gate) when gate is non-null. o, gate [S][Hq][256] (o may be null);
// with oq non-null also the Q8 quantization of o (oq [S][Hq * 256], os [S][Hq * 8]). At most 1024 items.
extern "C" __global__ void __launch_bounds__(256) halo_attn_decode_combine(
    const float* __restrict__ pm, const float* __restrict__ pl, const float* __restrict__ pacc,
    const float* __restrict__ gate, float* __restrict__ o, std::int8_t* __restrict__ oq, float* __restrict__ os,
    std::uint32_t S, std::uint32_t Hq, std::uint32_t Hkv, std::uint32_t prefix_chunks,
    std::uint32_t suffix_chunks) {
  __shared__ float wts[1024];
  __shared__ float red[4];
  const std::uint32_t G = Hq / Hkv, s = blockIdx.x / Hq, h = blockIdx.x % Hq, kvh = h / G, g = h % G;
  const std::uint32_t slot = s * G + g, slots = S * G, t = threadIdx.x;
  const std::uint32_t n = min(prefix_chunks + suffix_chunks, 1024u);
  auto item = [&](std::uint32_t i) -> std::size_t {
    const std::uint32_t c = i < prefix_chunks ? i : prefix_chunks + s * suffix_chunks + (i - prefix_chunks);
    return static_cast<std::size_t>(c) * Hkv + kvh;
  };
  float M = -INFINITY;
  for (std::uint32_t i = t; i < n; i += blockDim.x) {
    const float m = pm[item(i) * slots + slot];
    wts[i] = m;
    M = fmaxf(M, m);
  }
  M = halo::GroupMax(M);
  if (t % kWave == 0) red[t / kWave] = M;
  __syncthreads();
  M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float L = 0.0f;
  for (std::uint32_t i = t; i < n; i += blockDim.x) {
    const float m = wts[i];
    const float w = m == -INFINITY ? 0.0f : expf(m - M);
    wts[i] = w;
    L += w * pl[item(i) * slots + slot];
  }
  L = halo::GroupSum(L);
  __syncthreads();
  if (t % kWave == 0) red[t / kWave] = L;
  __syncthreads();
  L = (red[0] + red[1]) + (red[2] + red[3]);
  float acc = 0.0f;
  constexpr int kU = 8;
  for (std::uint32_t i0 = 0; i0 < n; i0 += kU) {
    float a[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const std::uint32_t i = min(i0 + u, n - 1);
      a[u] = wts[i] == 0.0f ? 0.0f : pacc[(item(i) * slots + slot) * kHd + t];
    }
#pragma unroll
    for (int u = 0; u < kU; ++u)
      if (i0 + u < n) acc += wts[i0 + u] * a[u];
  }
  float r = acc / L;
  const std::size_t off = (static_cast<std::size_t>(s) * Hq + h) * kHd + t;
  if (gate != nullptr) r *= halo::Sigmoid(gate[off]);
  if (o != nullptr) o[off] = r;
  if (oq != nullptr) {
    // the row's Q8 quantization for the output projection: 32-value blocks are half waves
    const float amax = halo::GroupMax<32>(fabsf(r));
    const float scale = amax / 127.0f;
    oq[off] = static_cast<std::int8_t>(scale > 0.0f ? static_cast<int>(rintf(r / scale)) : 0);
    if (t % 32 == 0) os[off / 32] = scale;
  }
}

// Appends one token's K and V per session at position nkv[s] - 1: k, v [S][Hkv][256] -> pools via page tables.
// grid (S * Hkv), block 64 (a float4 per lane).
extern "C" __global__ void __launch_bounds__(64)
    halo_kv_append(const float* __restrict__ k, const float* __restrict__ v, float* __restrict__ kpool,
                   float* __restrict__ vpool, const std::uint32_t* __restrict__ pages,
                   const std::uint32_t* __restrict__ nkv, std::uint32_t Hkv, std::uint32_t max_pages) {
  const std::uint32_t s = blockIdx.x / Hkv, kvh = blockIdx.x % Hkv, pos = nkv[s] - 1;
  const std::uint32_t pg = pages[static_cast<std::size_t>(s) * max_pages + pos / kPage];
  const std::size_t dst = ((static_cast<std::size_t>(pg) * Hkv + kvh) * kPage + pos % kPage) * kHd;
  const std::size_t src = (static_cast<std::size_t>(s) * Hkv + kvh) * kHd;
  reinterpret_cast<float4*>(kpool + dst)[threadIdx.x] = reinterpret_cast<const float4*>(k + src)[threadIdx.x];
  reinterpret_cast<float4*>(vpool + dst)[threadIdx.x] = reinterpret_cast<const float4*>(v + src)[threadIdx.x];
}
