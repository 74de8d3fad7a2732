// Workspace layout of the device sampler, shared by the kernels and the host dispatch (constexpr, so usable on
// both sides). Per launch of `rows` rows over a vocabulary of V tokens, nb = ceil(V / kSampleSlice) blocks per row:
//   val   [rows][V]  double  penalized logits, then (linear path) weights
//   fx    [rows][V]  u64     2^-40 fixed-point weights (wide kept sets)
//   pkey / ptok / pnf [rows][nb]         per-block best (DescKey, token) and finite count
//   psum / pnz / plast / pminw [rows][nb] per-block weight sum, nonzero count, last nonzero index + 1, least nonzero
//   hist  [rows][kSampleBins] u32        histogram of max - v
//   ckey / ctok [rows][kSampleCap], cn [rows]  collected candidates
#pragma once

#include <cstddef>
#include <cstdint>

namespace halo::sample {

constexpr std::uint32_t kSampleSlice = 4096;
constexpr std::uint32_t kSampleBins = 4096;
constexpr std::uint32_t kSampleCap = 4096;

struct Layout {
  std::size_t val, fx, pkey, ptok, pnf, psum, pnz, plast, pminw, hist, ckey, ctok, cn, bytes;
};

constexpr std::size_t Align256(std::size_t b) { return (b + 255) / 256 * 256; }
constexpr std::uint32_t Blocks(std::uint32_t V) { return (V + kSampleSlice - 1) / kSampleSlice; }

constexpr Layout MakeLayout(std::uint32_t rows, std::uint32_t V) {
  const std::size_t r = rows, v = V, nb = Blocks(V);
  Layout l{};
  std::size_t o = 0;
  l.val = o;   o += Align256(r * v * 8);
  l.fx = o;    o += Align256(r * v * 8);
  l.pkey = o;  o += Align256(r * nb * 8);
  l.ptok = o;  o += Align256(r * nb * 4);
  l.pnf = o;   o += Align256(r * nb * 4);
  l.psum = o;  o += Align256(r * nb * 8);
  l.pnz = o;   o += Align256(r * nb * 4);
  l.plast = o; o += Align256(r * nb * 4);
  l.pminw = o; o += Align256(r * nb * 8);
  l.hist = o;  o += Align256(r * kSampleBins * 4);
  l.ckey = o;  o += Align256(r * kSampleCap * 8);
  l.ctok = o;  o += Align256(r * kSampleCap * 4);
  l.cn = o;    o += Align256(r * 4);
  l.bytes = o;
  return l;
}

}  // namespace halo::sample
