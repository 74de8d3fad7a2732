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

using halo::H4;
using halo::H8;
using halo::Mfma3;
using halo::SplitHalves;
using halo::V4F;
namespace {
// Operand scales of the split-fp16 paths (powers of two, undone on the results): q and k (RMS-normalized) and V by 2^8,
// so values down to 2^-11 keep the full 22-bit split; a group (query row, K or V chunk) with a magnitude of 255.875 or
// more takes a smaller power of two instead (halo::SplitScale), keeping it in the fp16 range. The probabilities (<= 1)
// by 2^14.
constexpr float kSqk = 256.0f, kSvv = 256.0f, kSpp = 16384.0f;
constexpr float kLog2e = 1.4426950408889634f;
}  // namespace

// grid (Hkv * (prefix_chunks + S * suffix_chunks)), block 256.
//   q [S][Hq][256]; kpool, vpool [pages][Hkv][16][256]; pages [S][max_pages]; nkv [S] visible positions;
//   partial m, l [items][S * G], acc [items][S * G][256] (item = blockIdx.x).
// Prefix chunks cover tokens [32 c, 32 c + 32) < prefix of every session; suffix chunk c of session s covers
// [prefix + 32 c, ...) up to nkv[s]; positions at or past nkv[s] are masked, empty chunks record m = -inf.
//
// Every K and V load of the chunk (64 KB) is issued before any arithmetic, so a block keeps its whole chunk in
// flight. Scores: 16-lane row r of the block owns tokens r and r + 16, lane `sub` of the row dims
// {4 (16 u + sub) .. +4 : u < 4} (each load instruction reads 256 contiguous bytes per row); the 16 partial dots
// are summed with row DPP. V arrives as 16-byte loads and is staged through LDS (over the queries, once the scores
// are done). Weighted V: thread = one of the 256 dims, all 32 tokens in registers.
namespace {
// The partial kernel's body. kFused: q arrives as the raw q | gate projection qg [S][Hq][2 * 256] and is RMSNormed
// (wq) and rotated here at each session's position nkv[s] - 1, and the block whose chunk holds a session's newest
// position (the last suffix chunk) forms that position's K (RMSNorm wk, rotation) and V from kin / vin [S][Hkv][256],
// appends them to the pools and uses them for that row: the prologue launch before the attention disappears. The
// arithmetic is halo_attn_prep_decode's (halo::NormRopeHead), so q, K and V carry the same bits.
template <bool kFused, int kQW = 1, bool kMma = false>
__device__ __forceinline__ void AttnDecodePartial(
    const float* __restrict__ q, const float* __restrict__ kin, const float* __restrict__ vin,
    const float* __restrict__ wq, const float* __restrict__ wk, float* __restrict__ kpool, float* __restrict__ vpool,
    const std::uint32_t* __restrict__ pages, const std::uint32_t* __restrict__ nkv, float* __restrict__ pm,
    float* __restrict__ pl, float* __restrict__ pacc, std::uint32_t S, std::uint32_t Hq, std::uint32_t Hkv,
    std::uint32_t prefix, std::uint32_t max_pages, std::uint32_t prefix_chunks, std::uint32_t suffix_chunks,
    std::uint32_t rot, float theta, float eps) {
  // 32.5 KB: the queries, then the K chunk as halves, then the V chunk as halves (39 KB in all: four blocks per CU);
  // query rows padded by 16 bytes so the 16 rows of a matrix-core operand read fall on different banks
  __shared__ __attribute__((aligned(16))) float qs[kMaxQ][kHd + 4];
  __shared__ __attribute__((aligned(16))) float sc[kMaxQ][kChunk + 4];  // rows 16-byte aligned: vector reads
  static_assert(kChunk == 32 && kPage == 16, "two pages per chunk, two tokens per 16-lane row");
  const std::uint32_t G = Hq / Hkv, x = blockIdx.x, kvh = x % Hkv, c = x / Hkv;
  HALO_PHASE(1, 0);
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
  // the chunk's two pages (a position past the visible range reads the last visible one; it is masked)
  const std::uint32_t* pt = pages + static_cast<std::size_t>(sess) * max_pages;
  const std::uint32_t last = limit - 1;
  const std::uint32_t pg0 = pt[min(start, last) / kPage], pg1 = pt[min(start + kPage, last) / kPage];
  auto row_of = [&](const float* pool, std::uint32_t j) {  // token start + j, clamped to the visible range
    const std::uint32_t tok = min(start + j, last);
    const std::uint32_t pg = (tok - start) < kPage ? pg0 : pg1;
    return pool + ((static_cast<std::size_t>(pg) * Hkv + kvh) * kPage + tok % kPage) * kHd;
  };
  const std::uint32_t sub = t % 16, r = t / 16;
  // Fused prologue inputs, all issued before the chunk's K / V (a load issued after them could only be waited for
  // behind them): this wave's queries (kQW of them, slots past nq reload the last), their sessions' positions,
  // the norm weights and the newest position's k / v (loaded by every block, used by the one that holds it).
  static_assert(kQW >= 1 && kQW <= kMaxQ / 4, "queries per wave");
  float xq[kQW][4], wqv[4], wkv[4], xk[4], xv[4];
  std::uint32_t qpos[kQW];
  const bool owner = kFused && !is_prefix && last - start < static_cast<std::uint32_t>(kChunk);
  if constexpr (kFused) {
#pragma unroll
    for (int m = 0; m < kQW; ++m) {
      const std::uint32_t qi = min(wave + 4u * m, nq - 1);
      const std::uint32_t s = is_prefix ? qi / G : sess, g = is_prefix ? qi % G : qi;
      const float* src = q + (static_cast<std::size_t>(s) * Hq + kvh * G + g) * 2 * kHd;
#pragma unroll
      for (int i = 0; i < 4; ++i) xq[m][i] = src[lane + 64 * i];
      qpos[m] = nkv[s] - 1;
    }
    const std::size_t kv_src = (static_cast<std::size_t>(sess) * Hkv + kvh) * kHd;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      wqv[i] = wq[lane + 64 * i];
      wkv[i] = wk[lane + 64 * i];
      xk[i] = kin[kv_src + lane + 64 * i];
      xv[i] = vin[kv_src + lane + 64 * i];
    }
  }
  float4 kf[2][4];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float4* kr = reinterpret_cast<const float4*>(row_of(kpool, r + 16 * h));
#pragma unroll
    for (int u = 0; u < 4; ++u) kf[h][u] = kr[16 * u + sub];
  }
  // The V chunk (fused prologue: issued only after the query prologue; a wave's loads issue in order and stall while
  // the stream is queued, so V issued with K would hold that prologue back, and V is needed only after the scores)
  float4 vq[2][4];
  const std::uint32_t vdg = t % 64, vkg = t / 64;
  float4 vreg[8];
  auto issue_v = [&]() {
  if constexpr (!kMma) {
  // V as 16-byte loads of the two pages (each page's 16 rows are 16 KB contiguous; thread t takes float4 t of every
  // 4 KB part: row 4 part + t / 64, dims 4 (t % 64) ..): 4-byte loads of a column would take 32 instructions per
  // thread and run the chunk's V stream at half the rate. Staged through LDS below, so the weighted sum still reads
  // one dim of every row.
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float4* vp = reinterpret_cast<const float4*>(vpool + (static_cast<std::size_t>(h ? pg1 : pg0) * Hkv + kvh) *
                                                                   kPage * kHd);
#pragma unroll
    for (int u = 0; u < 4; ++u) vq[h][u] = vp[u * 256 + t];
  }
  } else {
  // V: thread t takes keys 8 (t / 64) + e (e < 8, one page) at dims 4 (t % 64) ..: each load instruction reads one
  // whole 1 KB row; staged transposed below (positions past the visible range are zeroed there)
  {
    const float* vp = vpool + ((static_cast<std::size_t>(vkg < 2 ? pg0 : pg1) * Hkv + kvh) * kPage) * kHd + 4 * vdg;
#pragma unroll
    for (int e = 0; e < 8; ++e) vreg[e] = *reinterpret_cast<const float4*>(vp + ((8 * vkg + e) % kPage) * kHd);
  }
  }
  };
  if constexpr (!kFused && !kMma) issue_v();
  // queries of this kv head: slot i = session * G + g (prefix) or g (suffix)
  __shared__ __attribute__((aligned(16))) float knew[kFused ? 2 : 1][kFused ? kHd : 4];
  if constexpr (kFused) {
    // wave w prepares queries w, w + 4, ... (the angles once per position)
    std::uint32_t cur = 0xFFFFFFFFu;
    halo::RopeCS cs{};
    float out[4];
#pragma unroll
    for (int m = 0; m < kQW; ++m) {
      const std::uint32_t qi = wave + 4u * m;
      if (qi >= nq) break;
      if (qpos[m] != cur) {
        cur = qpos[m];
        cs = halo::RopeAngles(cur, rot, theta);
      }
      halo::NormRopeHead(xq[m], wqv, cs, rot, eps, out);
#pragma unroll
      for (int i = 0; i < 4; ++i) qs[qi][lane + 64 * i] = out[i];
    }
    if (owner && wave == 3) {
      // the newest position's K and V: to LDS for this block's scores and weighted sum, and to the pools (its page
      // is one of the chunk's two)
      if (cur != last) cs = halo::RopeAngles(last, rot, theta);
      halo::NormRopeHead(xk, wkv, cs, rot, eps, out);
      const std::size_t dst =
          ((static_cast<std::size_t>(last - start < kPage ? pg0 : pg1) * Hkv + kvh) * kPage + last % kPage) * kHd;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        knew[0][lane + 64 * i] = out[i];
        knew[1][lane + 64 * i] = xv[i];
        kpool[dst + lane + 64 * i] = out[i];
        vpool[dst + lane + 64 * i] = xv[i];
      }
    }
  } else {
    for (std::uint32_t i = t; i < nq * (kHd / 4); i += blockDim.x) {
      const std::uint32_t qi = i / (kHd / 4), d4 = i % (kHd / 4);
      const std::uint32_t s = is_prefix ? qi / G : sess, g = is_prefix ? qi % G : qi;
      const float4 v = reinterpret_cast<const float4*>(q + (static_cast<std::size_t>(s) * Hq + kvh * G + g) * kHd)[d4];
      reinterpret_cast<float4*>(&qs[qi][0])[d4] = v;
    }
  }
  if constexpr (kFused && !kMma) issue_v();
  if constexpr (!kMma) {
  __syncthreads();
  HALO_PHASE(1, 1);
  if (owner) {
    // the newest row's K from LDS in place of the pool's (not yet written when the loads were issued)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      if (start + r + 16 * h == last)
#pragma unroll
        for (int u = 0; u < 4; ++u) kf[h][u] = reinterpret_cast<const float4*>(&knew[0][0])[16 * u + sub];
  }
  const float scale = 1.0f / sqrtf(static_cast<float>(kHd));
  const bool live0 = start + r < limit, live1 = start + r + 16 < limit;
  // queries in groups of 8, the group's dot products and row reductions interleaved (independent chains; each
  // query's arithmetic is the same as one at a time)
  constexpr int kQG = 8;
  for (std::uint32_t i0 = 0; i0 < nq; i0 += kQG) {
    float s0[kQG], s1[kQG];
#pragma unroll
    for (int k = 0; k < kQG; ++k) {
      const float4* qv = reinterpret_cast<const float4*>(&qs[min(i0 + k, nq - 1)][0]);
      s0[k] = 0.0f;
      s1[k] = 0.0f;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float4 b = qv[16 * u + sub];
        s0[k] += kf[0][u].x * b.x + kf[0][u].y * b.y + kf[0][u].z * b.z + kf[0][u].w * b.w;
        s1[k] += kf[1][u].x * b.x + kf[1][u].y * b.y + kf[1][u].z * b.z + kf[1][u].w * b.w;
      }
    }
#pragma unroll
    for (int k = 0; k < kQG; ++k) {
      s0[k] = halo::GroupSum<16>(s0[k]);
      s1[k] = halo::GroupSum<16>(s1[k]);
    }
    if (sub == 0)
#pragma unroll
      for (int k = 0; k < kQG; ++k)
        if (i0 + k < nq) {
          sc[i0 + k][r] = live0 ? s0[k] * scale : -INFINITY;
          sc[i0 + k][r + 16] = live1 ? s1[k] * scale : -INFINITY;
        }
  }
  __syncthreads();  // the scores are in sc and qs is free: the V rows go there (rows past the visible range as 0)
  HALO_PHASE(1, 2);
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const std::uint32_t j = 16 * h + 4 * u + t / 64;
      float4 v = start + j < limit ? vq[h][u] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (owner && start + j == last) v = reinterpret_cast<const float4*>(&knew[1][0])[t % 64];
      reinterpret_cast<float4*>(&qs[j][0])[t % 64] = v;
    }
  // softmax over the chunk per query: wave w takes queries w, w + 4, ...; lanes 0..31 are the tokens
  for (std::uint32_t i = wave; i < nq; i += 4) {
    const float s = lane < kChunk ? sc[i][lane] : -INFINITY;
    const float m = halo::GroupMax(s);
    const float p = s == -INFINITY ? 0.0f : expf(s - m);
    const float l = halo::GroupSum(p);
    if (lane < kChunk) sc[i][lane] = p;
    if (lane == 0) {
      const std::uint32_t slot = is_prefix ? i : sess * G + i;
      m_out[slot] = m;
      l_out[slot] = l;
    }
  }
  __syncthreads();
  HALO_PHASE(1, 3);
  // weighted V, 8 queries' sums interleaved (each still adds its tokens in order j = 0 .. 31); V and the weights
  // are read from LDS four tokens at a time
  for (std::uint32_t i0 = 0; i0 < nq; i0 += kQG) {
    float acc[kQG];
#pragma unroll
    for (int k = 0; k < kQG; ++k) acc[k] = 0.0f;
#pragma unroll 2
    for (int j4 = 0; j4 < kChunk; j4 += 4) {
      const float v0 = qs[j4][t], v1 = qs[j4 + 1][t], v2 = qs[j4 + 2][t], v3 = qs[j4 + 3][t];
#pragma unroll
      for (int k = 0; k < kQG; ++k) {
        const float4 p4 = *reinterpret_cast<const float4*>(&sc[min(i0 + k, nq - 1)][j4]);
        acc[k] += p4.x * v0;
        acc[k] += p4.y * v1;
        acc[k] += p4.z * v2;
        acc[k] += p4.w * v3;
      }
    }
#pragma unroll
    for (int k = 0; k < kQG; ++k)
      if (i0 + k < nq) {
        const std::uint32_t slot = is_prefix ? i0 + k : sess * G + i0 + k;
        a_out[static_cast<std::size_t>(slot) * kHd + t] = acc[k];
      }
  }
  HALO_PHASE(1, 4);
  } else {
  __syncthreads();
  HALO_PHASE(1, 1);
  // Matrix-core tiles: nqt tiles of 16 query rows (rows past nq repeat the last query and are never stored); the
  // scores are tiles (query tile w / 2, key tile w % 2) of waves w < 2 nqt; each query row's products, softmax and
  // weighted sum depend only on that row, so a query gets the same bits whichever block and batch it is scored in.
  const std::uint32_t nqt = (nq + 15) / 16, kq = lane / 16, lr = lane % 16;
  const std::uint32_t qt = wave / 2, kt = wave % 2;
  const bool score_wave = qt < nqt;
  // Operand scales (powers of two): per query row, and per block for the K and the V chunk (halo::SplitScale:
  // kSqk / kSvv unless the group's largest magnitude would overflow the fp16 range)
  __shared__ float qsc[kMaxQ], kvmax[2][4];
  H8 qh[kHd / 32], ql[kHd / 32];
  if (score_wave) {
    // two passes over the query row in LDS (its magnitude, then the split), so the row is never held in registers
    // next to its halves (that took the kernel to 180 VGPRs: two blocks per CU instead of three)
    const float* qr = &qs[min(16 * qt + lr, nq - 1)][0];
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < kHd / 32; ++c) {
      const float4 a0 = *reinterpret_cast<const float4*>(qr + 32 * c + 8 * kq);
      const float4 a1 = *reinterpret_cast<const float4*>(qr + 32 * c + 8 * kq + 4);
      amax = fmaxf(amax, fmaxf(fmaxf(fmaxf(fabsf(a0.x), fabsf(a0.y)), fmaxf(fabsf(a0.z), fabsf(a0.w))),
                               fmaxf(fmaxf(fabsf(a1.x), fabsf(a1.y)), fmaxf(fabsf(a1.z), fabsf(a1.w)))));
    }
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    const float sq = halo::SplitScale(amax, kSqk);
#pragma unroll
    for (int c = 0; c < kHd / 32; ++c) {
      const float4 a0 = *reinterpret_cast<const float4*>(qr + 32 * c + 8 * kq);
      const float4 a1 = *reinterpret_cast<const float4*>(qr + 32 * c + 8 * kq + 4);
      const float x[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
      SplitHalves(x, qh[c], ql[c], sq);
    }
    if (kq == 0) qsc[16 * qt + lr] = sq;
  }
  {  // the block's K and V magnitudes over the visible rows (rows past them repeat the pool's row `last`, which for
     // the owner block is not yet written: the newest row comes from LDS, and the masked rows' scores are dropped)
    float ka = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const std::uint32_t j = r + 16 * h;
      const bool fresh = owner && start + j == last;
      if (start + j < limit)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float4 kv = fresh ? *reinterpret_cast<const float4*>(&knew[0][64 * u + 4 * sub]) : kf[h][u];
          ka = fmaxf(ka, fmaxf(fmaxf(fabsf(kv.x), fabsf(kv.y)), fmaxf(fabsf(kv.z), fabsf(kv.w))));
        }
    }
    ka = halo::GroupMax(ka);
    if (lane == 0) kvmax[0][wave] = ka;
  }
  __syncthreads();  // qs is free: the K chunk goes there as halves
  const float sk = halo::SplitScale(fmaxf(fmaxf(kvmax[0][0], kvmax[0][1]), fmaxf(kvmax[0][2], kvmax[0][3])), kSqk);
  // K halves kh / kl [32 keys][256]: 16-byte chunk c of key row j at c ^ (j & 15) (the 16 lanes of an operand read
  // take 16 different bank groups); the newest row (owner) from LDS, not yet in the pool when it was loaded
  _Float16* kh = reinterpret_cast<_Float16*>(&qs[0][0]);
  _Float16* kl = kh + kChunk * kHd;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const std::uint32_t j = r + 16 * h;
    const bool fresh = owner && start + j == last;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const std::uint32_t dim = 64 * u + 4 * sub;
      const float4 kv = fresh ? *reinterpret_cast<const float4*>(&knew[0][dim]) : kf[h][u];
      const float x[4] = {kv.x, kv.y, kv.z, kv.w};
      const std::uint32_t off = j * kHd + 8 * ((dim / 8) ^ (j & 15)) + dim % 8;
      H4 hi, lo;
      halo::SplitHalves4(x, hi, lo, sk);
      *reinterpret_cast<H4*>(&kh[off]) = hi;
      *reinterpret_cast<H4*>(&kl[off]) = lo;
    }
  }
  __syncthreads();
  HALO_PHASE(1, 2);
  // the V chunk issued only now that the K fragments are in LDS (its 32 destination registers and the K fragments
  // are never live together: held together they spilled, and the spill's reloads waited for V before the K phase)
  issue_v();
  const float scale = 1.0f / sqrtf(static_cast<float>(kHd));
  if (score_wave) {
    V4F c4 = {0.0f, 0.0f, 0.0f, 0.0f};
    const std::uint32_t key = 16 * kt + lr;
#pragma unroll
    for (int c = 0; c < kHd / 32; ++c) {
      const std::uint32_t off = key * kHd + 8 * ((4 * c + kq) ^ (key & 15));
      c4 = Mfma3(qh[c], ql[c], *reinterpret_cast<const H8*>(&kh[off]), *reinterpret_cast<const H8*>(&kl[off]), c4);
    }
    // C tile: lane (key lr, kq) holds rows 16 qt + 4 kq + i
    const bool live = start + key < limit;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const std::uint32_t qi = 16 * qt + 4 * kq + i;
      if (qi < nq) sc[qi][key] = live ? c4[i] * (scale / (qsc[qi] * sk)) : -INFINITY;
    }
  }
  {  // the V chunk's magnitude over the visible rows (the newest row from LDS), only now that the scores are done
    float va = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const std::uint32_t j = 8 * vkg + e;
      float4 vv = vreg[e];
      if (owner && start + j == last) vv = *reinterpret_cast<const float4*>(&knew[kFused ? 1 : 0][4 * vdg]);
      if (start + j < limit)
        va = fmaxf(va, fmaxf(fmaxf(fabsf(vv.x), fabsf(vv.y)), fmaxf(fabsf(vv.z), fabsf(vv.w))));
    }
    va = halo::GroupMax(va);
    if (lane == 0) kvmax[1][wave] = va;
  }
  __syncthreads();
  HALO_PHASE(1, 3);
  const float sv = halo::SplitScale(fmaxf(fmaxf(kvmax[1][0], kvmax[1][1]), fmaxf(kvmax[1][2], kvmax[1][3])), kSvv);
  // the K chunk is done with: the V chunk goes to the same LDS as halves transposed, vh / vl [256 dims][32 keys]
  // (chunk c of 8 keys of a dim row at c ^ ((dim >> 2) & 3))
  _Float16* vh = kh;
  _Float16* vl = kh + kHd * kChunk;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const std::uint32_t dim = 4 * vdg + d;
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const std::uint32_t j = 8 * vkg + e;
      const float4 vv = vreg[e];
      float val = d == 0 ? vv.x : d == 1 ? vv.y : d == 2 ? vv.z : vv.w;
      if (owner && start + j == last) val = knew[kFused ? 1 : 0][dim];
      x[e] = start + j < limit ? val : 0.0f;
    }
    H8 hi, lo;
    SplitHalves(x, hi, lo, sv);
    const std::uint32_t off = dim * kChunk + 8 * (vkg ^ ((dim >> 2) & 3));
    *reinterpret_cast<H8*>(&vh[off]) = hi;
    *reinterpret_cast<H8*>(&vl[off]) = lo;
  }
  // softmax over the chunk per query: wave w takes queries w, w + 4, ...; lanes 0..31 are the tokens
  for (std::uint32_t i = wave; i < nq; i += 4) {
    const float s = lane < kChunk ? sc[i][lane] : -INFINITY;
    const float m = halo::GroupMax(s);
    const float p = s == -INFINITY ? 0.0f : expf(s - m);
    const float l = halo::GroupSum(p);
    if (lane < kChunk) sc[i][lane] = p;
    if (lane == 0) {
      const std::uint32_t slot = is_prefix ? i : sess * G + i;
      m_out[slot] = m;
      l_out[slot] = l;
    }
  }
  __syncthreads();
  HALO_PHASE(1, 5);
  // weighted V: output tiles (query tile, 16-dim tile); two query tiles: wave w takes tile w / 2, dim tiles
  // 8 (w % 2) ..; one: dim tiles 4 w .. + 3
  const std::uint32_t pqt = nqt == 2 ? wave / 2 : 0, ndt = nqt == 2 ? 8 : 4, dt0 = nqt == 2 ? 8 * (wave % 2) : 4 * wave;
  H8 pah, pal;
  {
    const float* pr = &sc[min(16 * pqt + lr, nq - 1)][8 * kq];
    const float4 a0 = *reinterpret_cast<const float4*>(pr), a1 = *reinterpret_cast<const float4*>(pr + 4);
    const float x[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    SplitHalves(x, pah, pal, kSpp);
  }
#pragma unroll
  for (std::uint32_t dc = 0; dc < 8; ++dc) {
    if (dc >= ndt) break;
    const std::uint32_t dim = 16 * (dt0 + dc) + lr;
    const std::uint32_t off = dim * kChunk + 8 * (kq ^ ((dim >> 2) & 3));
    const V4F acc = Mfma3(pah, pal, *reinterpret_cast<const H8*>(&vh[off]), *reinterpret_cast<const H8*>(&vl[off]),
                          V4F{0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const std::uint32_t qi = 16 * pqt + 4 * kq + i;
      if (qi < nq) {
        const std::uint32_t slot = is_prefix ? qi : sess * G + qi;
        a_out[static_cast<std::size_t>(slot) * kHd + dim] = acc[i] * (1.0f / (kSpp * sv));
      }
    }
  }
  HALO_PHASE(1, 4);
  }
}
}  // namespace

// (the matrix-core forms ask for 3 waves per SIMD, i.e. at most 168 VGPRs: three 4-wave blocks per CU; at 180 the
// 608 blocks of the 4-session C4 step ran in two rounds)
#define HALO_ATTN_PARTIAL(NAME, MMA)                                                                                   \
  extern "C" __global__ void __launch_bounds__(256, MMA ? 3 : 1) NAME(                                                \
      const float* __restrict__ q, const float* __restrict__ kpool, const float* __restrict__ vpool,                 \
      const std::uint32_t* __restrict__ pages, const std::uint32_t* __restrict__ nkv, float* __restrict__ pm,        \
      float* __restrict__ pl, float* __restrict__ pacc, std::uint32_t S, std::uint32_t Hq, std::uint32_t Hkv,      \
      std::uint32_t prefix, std::uint32_t max_pages, std::uint32_t prefix_chunks, std::uint32_t suffix_chunks) {    \
    AttnDecodePartial<false, 1, MMA>(q, nullptr, nullptr, nullptr, nullptr, const_cast<float*>(kpool),             \
                                     const_cast<float*>(vpool), pages, nkv, pm, pl, pacc, S, Hq, Hkv, prefix,      \
                                     max_pages, prefix_chunks, suffix_chunks, 0, 0.0f, 0.0f);                     \
  }
// fp32 VALU dot products (one session: eight queries per kv head, latency-bound) / split-fp16 matrix cores (several
// sessions: up to 32 queries per block score a shared-prefix chunk)
HALO_ATTN_PARTIAL(halo_attn_decode_partial, false)
HALO_ATTN_PARTIAL(halo_attn_decode_partial_mma, true)
#undef HALO_ATTN_PARTIAL

// The partial launch with the attention prologue folded in (see AttnDecodePartial<true>): qg [S][Hq][2 * 256],
// kin, vin [S][Hkv][256], wq, wk [256]; rot <= 128. Every session's newest position nkv[s] - 1 must lie past the
// shared prefix (it is in that session's last suffix chunk). Same grid and partial outputs as
// halo_attn_decode_partial; the gate for the combine is the second half of each qg head.
// _qk: up to 32 query vectors per block (S * Hq / Hkv <= 32), split-fp16 matrix cores; _qk2: up to 8 (two per
// wave), fp32 VALU.
#define HALO_ATTN_PARTIAL_QK(NAME, QW, MMA)                                                                           \
  extern "C" __global__ void __launch_bounds__(256, MMA ? 3 : 1) NAME(                                          \
      const float* __restrict__ qg, const float* __restrict__ kin, const float* __restrict__ vin,               \
      const float* __restrict__ wq, const float* __restrict__ wk, float* __restrict__ kpool,                    \
      float* __restrict__ vpool, const std::uint32_t* __restrict__ pages, const std::uint32_t* __restrict__ nkv, \
      float* __restrict__ pm, float* __restrict__ pl, float* __restrict__ pacc, std::uint32_t S, std::uint32_t Hq, \
      std::uint32_t Hkv, std::uint32_t prefix, std::uint32_t max_pages, std::uint32_t prefix_chunks,            \
      std::uint32_t suffix_chunks, std::uint32_t rot, float theta, float eps) {                                 \
    AttnDecodePartial<true, QW, MMA>(qg, kin, vin, wq, wk, kpool, vpool, pages, nkv, pm, pl, pacc, S, Hq, Hkv, prefix,  \
                                max_pages, prefix_chunks, suffix_chunks, rot, theta, eps);                       \
  }
HALO_ATTN_PARTIAL_QK(halo_attn_decode_partial_qk, 8, true)
HALO_ATTN_PARTIAL_QK(halo_attn_decode_partial_qk2, 2, false)
#undef HALO_ATTN_PARTIAL_QK


// grid (S * Hq * NS), block 256: block (s, h, slice) merges the partials of session s, head h over its prefix and
// suffix chunks (log-sum-exp) for the slice's 256 / NS dims: o = acc / l, then o *= sigmoid(gate) when gate is
// non-null. o, gate [S][Hq][256] (o may be null); with oq non-null also the Q8 quantization of o (oq [S][Hq * 256],
// os [S][Hq * 8]). At most 1024 items. Thread: float4 lane f of the slice, item group t / (lanes per slice), eight
// loads in flight. NS = 8 doubles the blocks of small batches (more loads in flight over the chip).
namespace {
template <int NS, int kGS = 1>
__device__ __forceinline__ void AttnDecodeCombine(
    const float* __restrict__ pm, const float* __restrict__ pl, const float* __restrict__ pacc,
    const float* __restrict__ gate, float* __restrict__ o, std::int8_t* __restrict__ oq, float* __restrict__ os,
    std::uint32_t S, std::uint32_t Hq, std::uint32_t Hkv, std::uint32_t prefix_chunks,
    std::uint32_t suffix_chunks) {
  constexpr std::uint32_t kW = kHd / NS, kF = kW / 4, kG = 256 / kF;  // slice dims, float4 lanes, item groups
  __shared__ float wts[1024];
  __shared__ float red[4], redl[4];
  __shared__ float4 part[kG][kF];
  const std::uint32_t quarter = blockIdx.x % NS, sh = blockIdx.x / NS;
  const std::uint32_t G = Hq / Hkv, s = sh / Hq, h = sh % Hq, kvh = h / G, g = h % G;
  const std::uint32_t slot = s * G + g, slots = S * G, t = threadIdx.x;
  const std::uint32_t n = min(prefix_chunks + suffix_chunks, 1024u);
  auto item = [&](std::uint32_t i) -> std::size_t {
    const std::uint32_t c = i < prefix_chunks ? i : prefix_chunks + s * suffix_chunks + (i - prefix_chunks);
    return static_cast<std::size_t>(c) * Hkv + kvh;
  };
  // The loads that do not depend on each other are issued together (unconditionally, from clamped items, then
  // selected): the items' m and l for n <= 512 (two each per thread), this thread's first group of kU partial sums
  // and its gate value; further items (n > 512, groups past the first) are loaded where they are used. The
  // arithmetic runs in the order it always had.
  const std::uint32_t f = t % kF, ig = t / kF;
  constexpr int kU = 8;
  float mv[2], lv[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const std::uint32_t i = min(t + 256u * j, n - 1);
    mv[j] = pm[item(i) * slots + slot];
    lv[j] = pl[item(i) * slots + slot];
  }
  float4 a0[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const std::uint32_t i = min(ig + kG * u, n - 1);
    a0[u] = reinterpret_cast<const float4*>(pacc + (item(i) * slots + slot) * kHd)[quarter * kF + f];
  }
  const float gv = *(gate != nullptr ? gate + (static_cast<std::size_t>(s) * Hq + h) * kGS * kHd + quarter * kW +
                                           min(t, kW - 1)
                                     : pl);  // (any valid address without a gate; unused then)
  const std::size_t off = (static_cast<std::size_t>(s) * Hq + h) * kHd + quarter * kW + min(t, kW - 1);
  float M = -INFINITY;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const std::uint32_t i = t + 256u * j;
    if (i < n) {
      wts[i] = mv[j];
      M = fmaxf(M, mv[j]);
    }
  }
  for (std::uint32_t i = t + 512; i < n; i += blockDim.x) {
    const float m = pm[item(i) * slots + slot];
    wts[i] = m;
    M = fmaxf(M, m);
  }
  M = halo::GroupMax(M);
  if (t % kWave == 0) red[t / kWave] = M;
  __syncthreads();
  M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float L = 0.0f;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const std::uint32_t i = t + 256u * j;
    if (i < n) {
      const float m = mv[j];
      const float w = m == -INFINITY ? 0.0f : expf(m - M);
      wts[i] = w;
      L += w * lv[j];
    }
  }
  for (std::uint32_t i = t + 512; i < n; i += blockDim.x) {
    const float m = wts[i];
    const float w = m == -INFINITY ? 0.0f : expf(m - M);
    wts[i] = w;
    L += w * pl[item(i) * slots + slot];
  }
  L = halo::GroupSum(L);
  if (t % kWave == 0) redl[t / kWave] = L;  // (its own array: red may still be read for M)
  __syncthreads();
  L = (redl[0] + redl[1]) + (redl[2] + redl[3]);
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (std::uint32_t i0 = ig, r = 0; i0 < n; i0 += kG * kU, ++r) {
    float4 b[kU];
    float w[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const std::uint32_t i = i0 + kG * u;
      const float wi = wts[min(i, n - 1)];
      w[u] = i < n ? wi : 0.0f;
      // past the preloaded group: load here (clamped item); an empty chunk's partial is never written
      const float4 av = r == 0 ? a0[u]
                               : reinterpret_cast<const float4*>(pacc + (item(min(i, n - 1)) * slots + slot) *
                                                                           kHd)[quarter * kF + f];
      b[u] = w[u] == 0.0f ? make_float4(0.0f, 0.0f, 0.0f, 0.0f) : av;
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      acc.x += w[u] * b[u].x;
      acc.y += w[u] * b[u].y;
      acc.z += w[u] * b[u].z;
      acc.w += w[u] * b[u].w;
    }
  }
  part[ig][f] = acc;
  __syncthreads();
  if (t >= kW) return;
  // lane = dim of the slice
  float sum = 0.0f;
#pragma unroll
  for (std::uint32_t k = 0; k < kG; ++k) sum += reinterpret_cast<const float*>(&part[k][0])[t];
  float r = sum / L;
  if (gate != nullptr) r *= halo::Sigmoid(gv);
  if (o != nullptr) o[off] = r;
  if (oq != nullptr) {
    // the row's Q8 quantization for the output projection: 32-value blocks are half waves
    const float amax = halo::GroupMax<32>(fabsf(r));
    const float scale = amax / 127.0f;
    oq[off] = static_cast<std::int8_t>(scale > 0.0f ? static_cast<int>(rintf(r / scale)) : 0);
    if (t % 32 == 0) os[off / 32] = scale;
  }
}
}  // namespace

// _qg: gate rows with a head stride of 2 * 256 (the gate halves of the q | gate projection, gate = qg + 256).
#define HALO_ATTN_COMBINE(NAME, NS, GS)                                                                          \
  extern "C" __global__ void __launch_bounds__(256) NAME(                                                       \
      const float* __restrict__ pm, const float* __restrict__ pl, const float* __restrict__ pacc,               \
      const float* __restrict__ gate, float* __restrict__ o, std::int8_t* __restrict__ oq, float* __restrict__ os, \
      std::uint32_t S, std::uint32_t Hq, std::uint32_t Hkv, std::uint32_t prefix_chunks,                         \
      std::uint32_t suffix_chunks) {                                                                             \
    AttnDecodeCombine<NS, GS>(pm, pl, pacc, gate, o, oq, os, S, Hq, Hkv, prefix_chunks, suffix_chunks);         \
  }
HALO_ATTN_COMBINE(halo_attn_decode_combine, 4, 1)
HALO_ATTN_COMBINE(halo_attn_decode_combine8, 8, 1)
HALO_ATTN_COMBINE(halo_attn_decode_combine_qg, 4, 2)
HALO_ATTN_COMBINE(halo_attn_decode_combine8_qg, 8, 2)
#undef HALO_ATTN_COMBINE

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

// ---- causal GQA attention for a ragged batch of prefill tokens (split-fp16 MFMA) -----------------------------------
// Reference semantics: ReferenceModel::Attention (src/model/reference.cpp:368-416, 492-527) for every token of a
// prompt: softmax(q . K[0..p]^T / sqrt(d)) V[0..p] * sigmoid(gate), K / V already appended at the tokens' positions.
// tiles [n][4] = {first token index in the batch, tokens (<= 8), session, position of the first token}; a tile's
// tokens are consecutive positions of one session. Block (tile, kv head): 64 queries = 8 tokens x G = 8 q heads,
// wave w the tokens 2w, 2w + 1 (query row r = 8 (token - 2w) + g). Per 32-key chunk: scores on
// the matrix cores (A = q rows kept in registers, B = K chunk in LDS), online softmax per row in the MFMA output
// layout (a row's 32 scores sit in one 16-lane DPP row, two tiles), P through LDS, P V with the same MFMA (B = V
// chunk in LDS). Output o (fp32, may be null) and its Q8 quantization oq / os (may be null), per token
// [Hq * 256], after o /= l and o *= sigmoid(gate). q, gate [T][Hq][256].
//
// Every fp32 operand x enters as a pair of halves, hi = fp16(x) and lo = fp16(x - hi) (|x - hi - lo| <= 2^-22 |x|
// for normal values), and each product is formed as hi * hi + hi * lo + lo * hi on v_mfma_f32_16x16x32_f16
// (products of halves are exact in the fp32 accumulator; the dropped lo * lo term is below 2^-22 of the product).
// Three fp16 MFMAs cost 3/16 of the fp32 MFMA issue time of the same products, so the scores and P V run at about
// five times the fp32 MFMA rate with fp32-level accuracy. q, k and V are scaled by 2^8 and the probabilities by 2^14
// before the split (kSqk, kSvv, kSpp); a query row, K chunk or V chunk whose magnitude would overflow fp16 at 2^8
// takes a smaller power of two (halo::SplitScale), so any finite operand range is accepted.
// (An fp32 version of this kernel on v_mfma_f32_16x16x4f32 ran the C4 prefix prefill's attention at 78.8 TFLOP/s.)
// The K and V chunks are converted once per block while staged in LDS: K as kh / kl [key][256] (16-byte chunk c of row key at
// c ^ (key & 15): the 16 lanes reading one column of keys hit 16 different bank groups), V transposed as vh / vl
// [dim][32 keys] (chunk c at c ^ ((dim >> 2) & 3)), so each MFMA operand is one 16-byte LDS read. The next chunk's
// K and V are loaded into registers while the current chunk computes.

extern "C" __global__ void __launch_bounds__(256, 2) halo_attn_prefill(
    const float* __restrict__ q, const float* __restrict__ gate, const float* __restrict__ kpool,
    const float* __restrict__ vpool, const std::uint32_t* __restrict__ pages, const std::uint32_t* __restrict__ tiles,
    float* __restrict__ o, std::int8_t* __restrict__ oq, float* __restrict__ os, std::uint32_t Hq, std::uint32_t Hkv,
    std::uint32_t max_pages) {
  __shared__ __attribute__((aligned(16))) _Float16 kh[kChunk * kHd], kl[kChunk * kHd];
  __shared__ __attribute__((aligned(16))) _Float16 vh[kHd * kChunk], vl[kHd * kChunk];
  __shared__ __attribute__((aligned(16))) _Float16 ph[4][16 * kChunk], pl[4][16 * kChunk];
  const std::uint32_t G = Hq / Hkv;
  const std::uint32_t* tl = tiles + 4 * static_cast<std::size_t>(blockIdx.x);
  const std::uint32_t first = tl[0], ntok = tl[1], sess = tl[2], p0 = tl[3];
  const std::uint32_t kvh = blockIdx.y;
  const std::uint32_t t = threadIdx.x, wave = t / kWave, lane = t % kWave;
  const std::uint32_t row = lane % 16, kq = lane / 16;
  const std::uint32_t last = p0 + ntok - 1;
  const std::uint32_t nchunks = last / kChunk + 1;
  const std::uint32_t* pt = pages + static_cast<std::size_t>(sess) * max_pages;
  // staging roles: K rows key = t / 8, 32-byte pieces part + 8 j; V keys 8 (t / 64) + e at dims 4 (t % 64) ..
  const std::uint32_t skey = t / 8, spart = t % 8, vdg = t % 64, vkg = t / 64;
  float4 kreg[8], vreg[8];
  auto load_chunk = [&](std::uint32_t k0) {
    {
      const std::uint32_t kp = min(k0 + skey, last);
      const float4* ks = reinterpret_cast<const float4*>(
          kpool + ((static_cast<std::size_t>(pt[kp / kPage]) * Hkv + kvh) * kPage + kp % kPage) * kHd);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        kreg[2 * j] = ks[2 * (spart + 8 * j)];
        kreg[2 * j + 1] = ks[2 * (spart + 8 * j) + 1];
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const std::uint32_t kp = min(k0 + 8 * vkg + e, last);
      vreg[e] = reinterpret_cast<const float4*>(
          vpool + ((static_cast<std::size_t>(pt[kp / kPage]) * Hkv + kvh) * kPage + kp % kPage) * kHd)[vdg];
    }
  };
  auto stage_chunk = [&](float sk, float sv) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float x[8] = {kreg[2 * j].x,     kreg[2 * j].y,     kreg[2 * j].z,     kreg[2 * j].w,
                          kreg[2 * j + 1].x, kreg[2 * j + 1].y, kreg[2 * j + 1].z, kreg[2 * j + 1].w};
      H8 hi, lo;
      SplitHalves(x, hi, lo, sk);
      const std::uint32_t off = skey * kHd + 8 * ((spart + 8 * j) ^ (skey & 15));
      *reinterpret_cast<H8*>(&kh[off]) = hi;
      *reinterpret_cast<H8*>(&kl[off]) = lo;
    }
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = d == 0 ? vreg[e].x : d == 1 ? vreg[e].y : d == 2 ? vreg[e].z : vreg[e].w;
      H8 hi, lo;
      SplitHalves(x, hi, lo, sv);
      const std::uint32_t dim = 4 * vdg + d;
      const std::uint32_t off = dim * kChunk + 8 * (vkg ^ ((dim >> 2) & 3));
      *reinterpret_cast<H8*>(&vh[off]) = hi;
      *reinterpret_cast<H8*>(&vl[off]) = lo;
    }
  };
  load_chunk(0);
  // this lane's A-operand query: row r -> token 2 wave + r / 8, head r % 8; dims 32 c + 8 kq .. + 7
  const std::uint32_t qtok = min(2 * wave + row / 8, ntok - 1), qg = row % 8;
  const float* qrow = q + ((static_cast<std::size_t>(first) + qtok) * Hq + kvh * G + qg) * kHd;
  // Operand scales (powers of two, halo::SplitScale): per query row, per chunk for K; V's scale is the smallest of
  // the chunks so far (the accumulators are rescaled, exactly, when it drops)
  H8 qh[kHd / 32], ql[kHd / 32];
  float sqc[4];
  {
    float xr[kHd / 32][8];
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < kHd / 32; ++c) {
      const float4 a = *reinterpret_cast<const float4*>(qrow + 32 * c + 8 * kq);
      const float4 b = *reinterpret_cast<const float4*>(qrow + 32 * c + 8 * kq + 4);
      const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xr[c][e] = x[e];
        amax = fmaxf(amax, fabsf(x[e]));
      }
    }
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    const float sq = halo::SplitScale(amax, kSqk);
#pragma unroll
    for (int c = 0; c < kHd / 32; ++c) SplitHalves(xr[c], qh[c], ql[c], sq);
#pragma unroll
    for (int i = 0; i < 4; ++i) sqc[i] = __shfl(sq, 4 * kq + i);  // the scales of this lane's output rows
  }
  __shared__ float kvmax[2][4];
  float sv = kSvv;
  std::uint32_t qpos[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) qpos[i] = p0 + 2 * wave + (4 * kq + i) / 8;
  float m[4], l[4];
  V4F acc[kHd / 16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.0f;
  }
#pragma unroll
  for (int c = 0; c < kHd / 16; ++c) acc[c] = V4F{0.0f, 0.0f, 0.0f, 0.0f};
  const float scale = 1.0f / sqrtf(static_cast<float>(kHd));
  _Float16* pwh = &ph[wave][0];
  _Float16* pwl = &pl[wave][0];
  for (std::uint32_t ch = 0; ch < nchunks; ++ch) {
    const std::uint32_t k0 = ch * kChunk;
    {  // the chunk's K and V magnitudes
      float ka = 0.0f, va = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        ka = fmaxf(ka, fmaxf(fmaxf(fabsf(kreg[e].x), fabsf(kreg[e].y)), fmaxf(fabsf(kreg[e].z), fabsf(kreg[e].w))));
        va = fmaxf(va, fmaxf(fmaxf(fabsf(vreg[e].x), fabsf(vreg[e].y)), fmaxf(fabsf(vreg[e].z), fabsf(vreg[e].w))));
      }
      ka = halo::GroupMax(ka);
      va = halo::GroupMax(va);
      if (lane == 0) {
        kvmax[0][wave] = ka;
        kvmax[1][wave] = va;
      }
    }
    __syncthreads();  // every wave is done with the previous chunk's LDS
    const float sk = halo::SplitScale(fmaxf(fmaxf(kvmax[0][0], kvmax[0][1]), fmaxf(kvmax[0][2], kvmax[0][3])), kSqk);
    const float svc = halo::SplitScale(fmaxf(fmaxf(kvmax[1][0], kvmax[1][1]), fmaxf(kvmax[1][2], kvmax[1][3])), kSvv);
    const float vfac = svc < sv ? svc / sv : 1.0f;  // exact: both are powers of two
    sv = fminf(sv, svc);
    stage_chunk(sk, sv);
    __syncthreads();
    if (ch + 1 < nchunks) load_chunk(k0 + kChunk);  // in flight while this chunk computes
    // scores: two 16 x 16 tiles (keys k0 .. k0 + 15, k0 + 16 .. k0 + 31); B lane (key row, dims 32 c + 8 kq ..)
    V4F sc[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      V4F c4 = {0.0f, 0.0f, 0.0f, 0.0f};
      const std::uint32_t key = 16 * h + row;
#pragma unroll
      for (int c = 0; c < kHd / 32; ++c) {
        const std::uint32_t off = key * kHd + 8 * ((4 * c + kq) ^ (key & 15));
        const H8 bh = *reinterpret_cast<const H8*>(&kh[off]);
        const H8 bl = *reinterpret_cast<const H8*>(&kl[off]);
        c4 = Mfma3(qh[c], ql[c], bh, bl, c4);
      }
      sc[h] = c4;
    }
    // online softmax per output row (lanes 16 kq .. 16 kq + 15 hold one row's 32 scores)
    float alpha[4];
    // Scores and the running max in base-2 units (scale * log2(e) folded into the score scale), so each
    // exponential is one v_exp_f32 and a masked score (-inf) needs no select.
    bool rescale = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float f = scale * kLog2e / (sqc[i] * sk);
      float s0 = sc[0][i] * f, s1 = sc[1][i] * f;
      const std::uint32_t kp0 = k0 + row, kp1 = k0 + 16 + row;
      s0 = kp0 <= qpos[i] ? s0 : -INFINITY;
      s1 = kp1 <= qpos[i] ? s1 : -INFINITY;
      const float cm = halo::GroupMax<16>(fmaxf(s0, s1));
      const float mx = fmaxf(m[i], cm);
      const bool none = mx == -INFINITY;
      alpha[i] = none ? 1.0f : __builtin_amdgcn_exp2f(m[i] - mx);
      rescale |= alpha[i] != 1.0f;
      const float e0 = __builtin_amdgcn_exp2f(s0 - mx), e1 = __builtin_amdgcn_exp2f(s1 - mx);
      l[i] = l[i] * alpha[i] + halo::GroupSum<16>(e0 + e1);
      m[i] = mx;
      // P row 4 kq + i, keys row and 16 + row; 16-byte chunk c of a P row at c ^ (kq & 3) (row >> 2 == kq)
      const std::uint32_t pr = (4 * kq + i) * kChunk;
      std::uint32_t ph2, pl2;
      halo::SplitPair(e0, e1, kSpp, ph2, pl2);
      const std::uint32_t o0 = pr + 8 * ((row / 8) ^ kq) + row % 8, o1 = pr + 8 * ((2 + row / 8) ^ kq) + row % 8;
      pwh[o0] = __builtin_bit_cast(_Float16, static_cast<std::uint16_t>(ph2 & 0xFFFFu));
      pwl[o0] = __builtin_bit_cast(_Float16, static_cast<std::uint16_t>(pl2 & 0xFFFFu));
      pwh[o1] = __builtin_bit_cast(_Float16, static_cast<std::uint16_t>(ph2 >> 16));
      pwl[o1] = __builtin_bit_cast(_Float16, static_cast<std::uint16_t>(pl2 >> 16));
    }
    // the accumulators change only where some row's max moved (rare once the first chunks are in)
    if (__any(rescale) || vfac != 1.0f)
#pragma unroll
      for (int c = 0; c < kHd / 16; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[c][i] *= alpha[i] * vfac;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // P V: A = P (row = query, k = keys 8 kq ..), B = V (k = keys 8 kq .., col = dim 16 c + row)
    const std::uint32_t pa = row * kChunk + 8 * (kq ^ ((row >> 2) & 3));
    const H8 pah = *reinterpret_cast<const H8*>(&pwh[pa]);
    const H8 pal = *reinterpret_cast<const H8*>(&pwl[pa]);
#pragma unroll
    for (int c = 0; c < kHd / 16; ++c) {
      const std::uint32_t dim = 16 * c + row;
      const std::uint32_t off = dim * kChunk + 8 * (kq ^ ((dim >> 2) & 3));
      const H8 bh = *reinterpret_cast<const H8*>(&vh[off]);
      const H8 bl = *reinterpret_cast<const H8*>(&vl[off]);
      acc[c] = Mfma3(pah, pal, bh, bl, acc[c]);
    }
  }
  // epilogue: rows 4 kq + i, dims 16 c + row
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const std::uint32_t r = 4 * kq + i;
    const std::uint32_t tok = 2 * wave + r / 8, g = r % 8;
    const bool live = tok < ntok;
    const std::size_t base = ((static_cast<std::size_t>(first) + min(tok, ntok - 1)) * Hq + kvh * G + g) * kHd;
    const float inv = 1.0f / l[i] * (1.0f / (kSpp * sv));
#pragma unroll
    for (int c = 0; c < kHd / 16; c += 2) {
      const std::uint32_t d0 = 16 * c + row, d1 = 16 * (c + 1) + row;
      const float v0 = acc[c][i] * inv * halo::Sigmoid(gate[base + d0]);
      const float v1 = acc[c + 1][i] * inv * halo::Sigmoid(gate[base + d1]);
      if (live && o != nullptr) {
        o[base + d0] = v0;
        o[base + d1] = v1;
      }
      if (oq != nullptr) {
        const float amax = halo::GroupMax<16>(fmaxf(fabsf(v0), fabsf(v1)));
        const float qs = amax / 127.0f;
        if (live) {
          oq[base + d0] = static_cast<std::int8_t>(qs > 0.0f ? static_cast<int>(rintf(v0 / qs)) : 0);
          oq[base + d1] = static_cast<std::int8_t>(qs > 0.0f ? static_cast<int>(rintf(v1 / qs)) : 0);
          if (row == 0) os[(base + 16 * c) / 32] = qs;
        }
      }
    }
  }
}
