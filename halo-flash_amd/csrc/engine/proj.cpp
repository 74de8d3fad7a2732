// Grouped projections with a fused activation prologue (halo_proj_q8* kernels): one launch for up to four Q8_0
// matrices that read the same activation rows. Replaces the reference's [RMSNorm] + quantize + per-matrix
// FlashNextGpu::MatVec sequence (src/engine/flash_next_gpu.cpp:212-254).
#include <algorithm>

#include "engine.hpp"

using namespace halo::engine;

namespace {

// Fewest tokens for which the mode-Q projection runs on the int8 matrix cores (halo_proj_q8m_c*): beyond the v_dot4
// kernel's 8. Up to 8 tokens the model's batched step keeps the v_dot4 kernels, whose per-token bits equal the
// one-session step's (a batch gives the same tokens as its sessions run alone).
constexpr std::uint32_t kProjMfmaMinTokens = 9;

int ProjQ8Mfma(halo_engine* eng, const halo_q8_matrix* mats, float* const* ys, uint32_t n_mats,
               const halo_proj_input* in, uint32_t tokens, char* err, size_t errlen) {
  const std::uint32_t cols = mats[0].cols;
  if (in->xq == nullptr || in->xs == nullptr) return SetErr(err, errlen, "proj: mode Q needs xq / xs"), -1;
  for (std::uint32_t i = 0; i < n_mats; ++i) {
    const halo_q8_matrix& w = mats[i];
    if (w.qs == nullptr || w.d == nullptr || ys[i] == nullptr || w.rows == 0 || w.cols != cols || w.qstride != cols)
      return SetErr(err, errlen, "proj: matrix %u (%u x %u, qstride %u) does not match cols %u", i, w.rows, w.cols,
                    w.qstride, cols),
             -1;
  }
  std::uint32_t off[5] = {0, 0, 0, 0, 0};
  for (std::uint32_t i = 0; i < 4; ++i) off[i + 1] = off[i] + (i < n_mats ? CeilDiv(mats[i].rows, 16) : 0);
  auto mat = [&](std::uint32_t i) { return i < n_mats ? mats[i] : mats[0]; };
  auto out = [&](std::uint32_t i) { return i < n_mats ? ys[i] : ys[0]; };
  auto rows = [&](std::uint32_t i) { return i < n_mats ? mats[i].rows : 0u; };
  char name[32];
  std::snprintf(name, sizeof name, "halo_proj_q8m_c%u", cols / 1024);
  const halo_arg a[] = {Ptr(in->xq), Ptr(in->xs),
                        Ptr(mat(0).qs), Ptr(mat(0).d), Ptr(out(0)), Ptr(mat(1).qs), Ptr(mat(1).d), Ptr(out(1)),
                        Ptr(mat(2).qs), Ptr(mat(2).d), Ptr(out(2)), Ptr(mat(3).qs), Ptr(mat(3).d), Ptr(out(3)),
                        U32(rows(0)), U32(rows(1)), U32(rows(2)), U32(rows(3)), U32(off[1]), U32(off[2]), U32(off[3]),
                        U32(tokens)};
  return Launch(eng, name, D3(off[4]), D3(512), a, err, errlen);
}

}  // namespace

extern "C" int halo_op_proj_q8_grid(halo_engine* eng, const halo_q8_matrix* mats, float* const* ys,
                                    uint32_t n_mats, const halo_proj_input* in, uint32_t tokens, uint32_t grid_blocks,
                                    uint32_t lanes_per_row, char* err, size_t errlen) {
  if (mats == nullptr || ys == nullptr || in == nullptr || n_mats == 0 || n_mats > 4)
    return SetErr(err, errlen, "proj: 1..4 matrices with outputs and an input descriptor"), -1;
  if (tokens == 0 || tokens > 16) return SetErr(err, errlen, "proj: tokens %u not in 1..16", tokens), -1;
  const std::uint32_t cols = mats[0].cols;
  // Quantized rows (mode Q) of more tokens than the VALU kernel takes on int8 matrix cores when the row length is one
  // the MFMA kernel covers. Tuning overrides: tasks_per_wave = lanes_per_row = 1 selects the VALU kernel, = 2 the
  // MFMA kernel, at any token count they support.
  const bool force_valu = grid_blocks == 1 && lanes_per_row == 1, force_mfma = grid_blocks == 2 && lanes_per_row == 2;
  if (in->mode == HALO_PROJ_Q && tokens <= 16 && (tokens >= kProjMfmaMinTokens || force_mfma) && !force_valu &&
      (cols == 1024 || cols == 2048 || cols == 4096))
    return ProjQ8Mfma(eng, mats, ys, n_mats, in, tokens, err, errlen);
  if (force_valu || force_mfma) grid_blocks = lanes_per_row = 0;
  if (tokens == 0 || tokens > 8) return SetErr(err, errlen, "proj: tokens %u not in 1..8", tokens), -1;
  if (cols == 0 || cols % 32 != 0 || cols > 4096) return SetErr(err, errlen, "proj: cols %u unsupported", cols), -1;
  for (std::uint32_t i = 0; i < n_mats; ++i) {
    const halo_q8_matrix& w = mats[i];
    if (w.qs == nullptr || w.d == nullptr || ys[i] == nullptr || w.rows == 0 || w.cols != cols || w.qstride != cols)
      return SetErr(err, errlen, "proj: matrix %u (%u x %u, qstride %u) does not match cols %u", i, w.rows, w.cols,
                    w.qstride, cols),
             -1;
  }
  const char* letter = nullptr;
  switch (in->mode) {
    case HALO_PROJ_Q:
      if (in->xq == nullptr || in->xs == nullptr) return SetErr(err, errlen, "proj: mode Q needs xq / xs"), -1;
      letter = "q";
      break;
    case HALO_PROJ_F:
      if (in->x == nullptr) return SetErr(err, errlen, "proj: mode F needs x"), -1;
      letter = "f";
      break;
    case HALO_PROJ_N:
      if (in->x == nullptr || in->norm_w == nullptr) return SetErr(err, errlen, "proj: mode N needs x / norm_w"), -1;
      if (in->res_out != nullptr && in->res_out == in->x)
        return SetErr(err, errlen, "proj: res_out must not alias the residual it reads"), -1;
      letter = "n";
      break;
    case HALO_PROJ_G:
      if (in->x == nullptr || in->delta == nullptr || in->norm_w == nullptr || cols % 128 != 0)
        return SetErr(err, errlen, "proj: mode G needs x / delta (gate) / norm_w and cols %% 128 == 0"), -1;
      letter = "g";
      break;
    default:
      return SetErr(err, errlen, "proj: mode %u unknown", in->mode), -1;
  }
  if ((in->xq_out == nullptr) != (in->xs_out == nullptr))
    return SetErr(err, errlen, "proj: xq_out and xs_out go together"), -1;
  // Lanes per row: the fewest that cover a row in at most four 16-byte pieces per lane (measured: 32 lanes x 4
  // pieces beats 64 x 2 on 2048 columns; more rows in flight per wave instruction).
  std::uint32_t lpr = cols > 2048 ? 64 : (cols > 1024 ? 32 : 16);
  if (lanes_per_row != 0) {
    if (!(lanes_per_row == 16 || lanes_per_row == 32 || lanes_per_row == 64) || cols > 64 * lanes_per_row)
      return SetErr(err, errlen, "proj: %u lanes per row cannot cover %u columns", lanes_per_row, cols), -1;
    lpr = lanes_per_row;
  }
  const std::uint32_t nb = tokens == 1 ? 1 : tokens == 2 ? 2 : tokens <= 4 ? 4 : 8;
  const std::uint32_t rows_per_task = 64 / lpr;
  std::uint32_t off[5] = {0, 0, 0, 0, 0};
  for (std::uint32_t i = 0; i < 4; ++i)
    off[i + 1] = off[i] + (i < n_mats ? CeilDiv(mats[i].rows, rows_per_task) : 0);
  // Tasks per wave: a prologue that normalizes (modes N and G, T rows of residual + delta + weights from L2) is
  // amortized over more rows per block; a plain quantized copy (mode Q) or quantization (mode F) is cheap enough
  // for one task per wave, which keeps the most waves (and loads) in flight.
  std::uint32_t tpw = (in->mode == HALO_PROJ_N || in->mode == HALO_PROJ_G) ? 4 : 1;
  if (grid_blocks == 1 || grid_blocks == 2 || grid_blocks == 4) tpw = grid_blocks;  // tuning override
  // One token in mode N with rows of at most 2048 columns: the 8-wave kernel (halo_proj_q8w_*), whose waves 4-7
  // stream weights while waves 0-3 form the normalized row.
  const bool wide = in->mode == HALO_PROJ_N && tokens == 1 && lpr <= 32;
  const std::uint32_t blocks = CeilDiv(off[4], (wide ? 8 : 4) * tpw);
  auto mat = [&](std::uint32_t i) { return i < n_mats ? mats[i] : mats[0]; };
  auto out = [&](std::uint32_t i) { return i < n_mats ? ys[i] : ys[0]; };
  auto rows = [&](std::uint32_t i) { return i < n_mats ? mats[i].rows : 0u; };
  char name[64];
  if (wide)
    std::snprintf(name, sizeof name, "halo_proj_q8w_l%u_t%u", lpr, tpw);
  else
    std::snprintf(name, sizeof name, "halo_proj_q8%s_l%u_b%u_t%u", letter, lpr, nb, tpw);
  const halo_arg a[] = {Ptr(in->x), Ptr(in->delta), Ptr(in->norm_w), Ptr(in->res_out), Ptr(in->xq), Ptr(in->xs),
                        Ptr(in->xq_out), Ptr(in->xs_out),
                        Ptr(mat(0).qs), Ptr(mat(0).d), Ptr(out(0)), Ptr(mat(1).qs), Ptr(mat(1).d), Ptr(out(1)),
                        Ptr(mat(2).qs), Ptr(mat(2).d), Ptr(out(2)), Ptr(mat(3).qs), Ptr(mat(3).d), Ptr(out(3)),
                        U32(rows(0)), U32(rows(1)), U32(rows(2)), U32(rows(3)), U32(off[1]), U32(off[2]), U32(off[3]),
                        U32(off[4]), U32(tokens), U32(cols), Val(in->eps)};
  return Launch(eng, name, D3(blocks), D3(wide ? 512 : 256), a, err, errlen);
}

extern "C" int halo_op_proj_q8(halo_engine* eng, const halo_q8_matrix* mats, float* const* ys, uint32_t n_mats,
                               const halo_proj_input* in, uint32_t tokens, char* err, size_t errlen) {
  return halo_op_proj_q8_grid(eng, mats, ys, n_mats, in, tokens, 0, 0, err, errlen);
}

extern "C" int halo_op_proj_q8_pair(halo_engine* eng, const halo_q8_matrix* mats, float* const* ys, uint32_t n_first,
                                    const halo_proj_input* in, const halo_proj_input* in2, uint32_t tokens, char* err,
                                    size_t errlen) {
  if (mats == nullptr || ys == nullptr || in == nullptr || in2 == nullptr || n_first < 1 || n_first > 2)
    return SetErr(err, errlen, "proj pair: 1 or 2 matrices on the first input, one on the second"), -1;
  if (in->mode != HALO_PROJ_Q || in2->mode != HALO_PROJ_Q || in->xq == nullptr || in->xs == nullptr ||
      in2->xq == nullptr || in2->xs == nullptr)
    return SetErr(err, errlen, "proj pair: both inputs quantized (mode Q, xq and xs)"), -1;
  if (tokens < 2 || tokens > 16) return SetErr(err, errlen, "proj pair: tokens %u not in 2..16", tokens), -1;
  const std::uint32_t n = n_first + 1, cols = mats[0].cols, cols2 = mats[n_first].cols;
  for (std::uint32_t i = 0; i < n; ++i) {
    const halo_q8_matrix& w = mats[i];
    const std::uint32_t c = i < n_first ? cols : cols2;
    if (w.qs == nullptr || w.d == nullptr || ys[i] == nullptr || w.rows == 0 || w.cols != c || w.qstride != c)
      return SetErr(err, errlen, "proj pair: matrix %u (%u x %u, qstride %u) does not match cols %u", i, w.rows,
                    w.cols, w.qstride, c),
             -1;
  }
  const halo_q8_matrix& m1 = n_first == 2 ? mats[1] : mats[0];
  float* y1 = n_first == 2 ? ys[1] : ys[0];
  if (tokens >= kProjMfmaMinTokens) {  // int8 matrix cores, 16-row tasks (halo_proj_q8m2_c2x4)
    if (cols != 2048 || cols2 != 4096)
      return SetErr(err, errlen, "proj pair: cols %u / %u have no paired kernel at %u tokens", cols, cols2, tokens),
             -1;
    const std::uint32_t o1 = CeilDiv(mats[0].rows, 16), o2 = o1 + (n_first == 2 ? CeilDiv(mats[1].rows, 16) : 0);
    const halo_arg a[] = {Ptr(in->xq), Ptr(in->xs), Ptr(mats[0].qs), Ptr(mats[0].d), Ptr(ys[0]), Ptr(m1.qs),
                          Ptr(m1.d), Ptr(y1), U32(mats[0].rows), U32(n_first == 2 ? mats[1].rows : 0u), U32(o1),
                          U32(o2), Ptr(in2->xq), Ptr(in2->xs), Ptr(mats[n_first].qs), Ptr(mats[n_first].d),
                          Ptr(ys[n_first]), U32(mats[n_first].rows), U32(tokens)};
    return Launch(eng, "halo_proj_q8m2_c2x4", D3(o2 + CeilDiv(mats[n_first].rows, 16)), D3(512), a, err, errlen);
  }
  // lanes per row as the single-input kernel picks them; the pairs built are (32, 64), (32, 32) and (64, 64)
  auto lanes = [](std::uint32_t c) { return c > 2048 ? 64u : (c > 1024 ? 32u : 16u); };
  const std::uint32_t l1 = lanes(cols), l2 = lanes(cols2);
  if (cols % 32 != 0 || cols2 % 32 != 0 || cols > 4096 || cols2 > 4096 || l1 == 16 || l2 == 16 ||
      (l1 == 64 && l2 == 32))
    return SetErr(err, errlen, "proj pair: cols %u / %u have no paired kernel", cols, cols2), -1;
  const std::uint32_t nb = tokens == 2 ? 2 : tokens <= 4 ? 4 : 8;
  if (nb == 2 && !(l1 == 32 && l2 == 64))
    return SetErr(err, errlen, "proj pair: 2 tokens only with 32 x 64 lanes"), -1;
  const std::uint32_t o1 = CeilDiv(mats[0].rows, 64 / l1);
  const std::uint32_t o2 = o1 + (n_first == 2 ? CeilDiv(mats[1].rows, 64 / l1) : 0);
  const std::uint32_t o3 = CeilDiv(mats[n_first].rows, 64 / l2);
  const std::uint32_t nb1 = CeilDiv(o2, 4), blocks = nb1 + CeilDiv(o3, 4);
  char name[48];
  std::snprintf(name, sizeof name, "halo_proj_q8q2_l%ux%u_b%u", l1, l2, nb);
  const halo_arg a[] = {Ptr(in->xq), Ptr(in->xs), Ptr(mats[0].qs), Ptr(mats[0].d), Ptr(ys[0]), Ptr(m1.qs), Ptr(m1.d),
                        Ptr(y1), U32(mats[0].rows), U32(n_first == 2 ? mats[1].rows : 0u), U32(o1), U32(o2),
                        U32(cols), Ptr(in2->xq), Ptr(in2->xs), Ptr(mats[n_first].qs), Ptr(mats[n_first].d),
                        Ptr(ys[n_first]), U32(mats[n_first].rows), U32(o3), U32(cols2), U32(nb1), U32(tokens)};
  return Launch(eng, name, D3(blocks), D3(256), a, err, errlen);
}
