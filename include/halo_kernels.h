/* Kernels of the embedded gfx950 code object (halo_core_code_object), looked up by name with halo_kernel().
 *
 * Reference-named kernels keep the reference's parameter lists and grid conventions (src/kernels/core.hip,
 * src/kernels/batch_decode.hip) so that host code launching them by name is a drop-in; the MI355X kernels under
 * new names carry their own grid conventions, documented at their definitions. Every pointer is a device buffer,
 * every other parameter a by-value scalar (src/rt/device.hpp:8-11).
 *
 *   halo_repack_q8_0(const u8* raw, i8* qs, u16* d, u32 rows, u32 cols, u32 qstride)         core.hip:2126
 *   halo_quantize_q8_rows(const f32* x, i8* xq, f32* xd, u32 cols)            grid (T)        core.hip:3089
 *   halo_quantize_q8_rows8(const f32* x, i8* xq, f32* xd, u32 cols, u32 T)    grid ceil(T / 8) (8 rows per block)
 *   halo_quantize_q8_rows2(x0, xq0, xd0, cols0, x1, xq1, xd1, cols1, T)   grid (2 T): two inputs in one launch
 *   halo_q8x_cols(const f32* x, u32 xstride, u32 cols, i8* xq, f32* xs, i8* xq2, f32* xs2)   batch_decode.hip:201
 *   halo_gemv_q8r{,_r2,_r4}(const i8* qs, const u16* d, const f32* x, f32* y, u32 rows, u32 cols, u32 qstride)
 *                                                       grid ceil(rows / (8 R))              core.hip:2175,2429
 *   halo_gemv_q8r_i8{,x}_r{1,2,4}_b{1..8}(qs, d, xq, xs, xq2, xs2, y, rows, cols, qstride, ystride, groups, chunk)
 *                                                       grid (ceil(rows/(8R)) * groups, parts) batch_decode.hip:301
 *   halo_gemv_q8r_i8{,x}_dual_r{1,2,4}_b{1..8}(q1, d1, y1, rows1, qstride1, q2, d2, y2, rows2, qstride2, xq, xs, xq2,
 *     xs2, cols, blocks1, ystride1, ystride2, groups)   grid ((blocks1 + blocks2) * groups)   batch_decode.hip:310
 *   halo_gemv_q8r_dual(q1, d1, y1, rows1, qstride1, q2, d2, y2, rows2, qstride2, x, cols, blocks1)
 *                                                       grid (blocks1 + ceil(rows2 / 32))    core.hip:2960
 *   halo_gemv_q8r_{r4,r2}_b{1..8}{,_p,_s,_ps}(qs, d, x, y, rows, cols, qstride, xstride, ystride, groups)
 *     exact batched fp32-x GEMVs, every column = the single-column kernel's bits; xstride % 4 == 0
 *                                                       grid (ceil(rows / (8 R)) * groups)   batch_decode.hip:133
 *   halo_gemv_q8r_dual_b{1..8}{,_p,_s,_ps}(q1, d1, y1, rows1, qstride1, q2, d2, y2, rows2, qstride2, x, cols,
 *     blocks1, xstride, ystride1, ystride2, groups)   grid ((blocks1 + ceil(rows2 / 32)) * groups)  batch_decode.hip:160
 *   halo_gemv_q8a8_l{16,32,64}_r{1,2,4}_b{1,2,4,8}(qs, d, xq, xs, y, rows, cols, qstride, ystride)   new (MI355X)
 *   halo_q8_half_dots(qs, xq, i32* isum, rows, cols, qstride)                                  new (parity)
 *   reference-named decode kernels (core.hip:259-586, 2621, 3003-3063), same parameters and grids:
 *     halo_rmsnorm(x, w_all, y, d, eps, w_stride)            grid (vectors)
 *     halo_l2norm(x, d, eps)                                 grid (vectors)
 *     halo_rope_neox(x, head_dim, rotary_dim, pos, theta), halo_rope_neox_rows(x, head_dim, rotary_dim, pos0, heads,
 *       theta), halo_rope_neox_p(x, params, head_dim, rotary_dim, slot, scale, theta)      grid (heads)
 *     halo_add(y, x, n), halo_axpy(y, x, a, n), halo_silu_mul(g, up, n), halo_sigmoid_gate(x, gate, n),
 *       halo_copy(dst, src, n), halo_copy_at(dst, src, params, slot, stride, n)          grid-stride
 *     halo_split_qgate(qg, q, gate, hd)                      grid (heads)
 *     halo_conv_step(in, state, w, out, channels, kern)      one thread per channel
 *     halo_conv_l2norm(in, state, w, out, channels, kern, l2_channels, eps)   block = one head of channels
 *     halo_gdn_step(q, k, v, alpha, beta, a, dt, state, out, num_k_heads, d)   grid (v heads), block >= d
 *     halo_gdn_step_d128(..., state, out, num_k_heads), halo_gdn_step_d128_norm(..., state, norm_w, z, out,
 *       num_k_heads, eps, mode)                              grid (v heads), block 128
 *     halo_gated_norm(o, w, z, d, eps, mode)                 grid (heads)
 *     halo_attention_decode(q, kc, vc, gate, out, scores, num_heads, num_kv_heads, hd, n, max_n)   grid (heads)
 *     halo_attention_prefill(..., num_heads, num_kv_heads, hd, pos0, max_n)                  grid (heads, T)
 *   reference-named MoE / GEMV kernels (core.hip:2183-2211, 2362-2378, 2436-2458, 2988, 3313, 9263-9285, 9401,
 *   9642), same parameters and grids:
 *     halo_gemv_q8r_wide / _r4n(qs, d, x, y, rows, cols, qstride)        grid ceil(rows / 8) / ceil(rows / 32)
 *     halo_gemv_q8r_expert{,_r4}(qs, d, ids, x, y, slot, rows, cols, qstride)   expert ids[slot] of a stacked tensor
 *     halo_moe_down_q8r{,_r4}(qs, d, ids, h, part, rows, cols, qstride)  grid (ceil(rows / (8 R)), slots)
 *     halo_moe_combine{,_u}(part, weights, out, slots, n)               grid-stride; _u: slots <= 16
 *     halo_matvec_f32_rowblock{,_u}(w, x, y, rows, cols)                grid (rows)
 *     halo_matvec_f32_rowblock2{,_u}(wa, wb, x, ya, yb, rows, cols)     grid (2 rows)
 *     halo_quantize_q8_kblocked(x, xq, xd, cols, tokens)                grid (T): xq [cols/64][T][64], xd [cols/32][T]
 *     halo_router_topk_w(logits, ids, weights, n, k)                    1 block of 256; n <= 1024, k <= 16
 *   reference-named select attention, DeltaNet prefill and shared-expert kernels (core.hip:783-918, 3480-3662,
 *   9196-9343, 9418-9446, 9590-9636), same parameters and grids:
 *     halo_attention_select{,_b}(q, kc, vc, gate, visible, out, scores, params, num_heads, num_kv_heads, hd, max_n)
 *       n = params[5], rows visible[0 .. n)                            grid (heads); _rows: grid (heads, T)
 *     halo_gdn_step_d128_norm_r(...)  as halo_gdn_step_d128_norm        grid (v heads), block 128
 *     halo_gdn_prefill_d128_norm(..., tokens, qk_stride, v_stride, zo_stride)   grid (v heads), block 128
 *     halo_conv_l2norm_prefill(in, state, w, out, channels, kern, l2_channels, eps)   grid (heads, T), block d
 *     halo_conv_state_advance(in, state, channels, kern, tokens)        grid ceil(channels / 256)
 *     halo_conv_l2norm_prefill8(in, state, w, out, channels, tokens, l2_channels, eps)   kern 4; grid
 *       (ceil(channels / 128), ceil(T / 8)), block 128 (a partial last head of channels is masked)
 *     halo_shexp_gate_up{,_u}(gq, gd, uq, ud, gate_inp, x, h, sgate, rows, cols, qstride)   grid ceil(rows / 16)
 *     halo_shexp_down_combine{,_u}(dq, dd, hin, sgate, part, weights, slots, out, rows, cols, qstride)
 *                                                                       grid ceil(rows / 32)
 *     halo_router_rowblock_q8act(w, x, y, rows, cols, act)              grid max(rows, cols / 32)
 *   fused norm + RoPE and batched-column glue (core.hip:308-440, 587, 1123-1133, 4045, 4708; batch_decode.hip:1680):
 *     halo_split_qgate_norm_rope(qg, q, gate, w, eps, rotary_dim, pos0, heads, theta)  grid (T * heads), block hd
 *     halo_norm_rope_rows(x, w, eps, d, rotary_dim, pos0, heads, theta, cache)          grid (T * heads), block 256
 *     halo_rope_neox_blocks(x, head_dim, rotary_dim, b0, ratio, theta)                   grid (nblocks)
 *     halo_rmsnorm_rows(x, w_all, y, d, eps, w_stride, w_period)                         grid (vectors)
 *     halo_split_qgate_y / halo_rmsnorm_y / halo_rope_neox_p_y / halo_copy_at_y           grid (., B)
 *     halo_axpy_slot, halo_axpy_sigmoid, halo_axpy_sigmoid_rows, halo_scale_silu          grid-stride
 *   fp32 GEMMs y [T][rows] (core.hip:3767-3800, 5605-5680, 8975-9000): halo_gemm_f32_tiled(w, x, y, rows, cols,
 *     tokens) grid (ceil(T / 64), ceil(rows / 64)); halo_gemm_f32_rows(w, x, y, rows, cols) grid (ceil(rows / 8), T);
 *     halo_gemm_f32_narrow(same) grid (ceil(rows / 256), T), cols <= 8192; halo_gemm_f32_skinny(w, x, y, rows, cols,
 *     tokens) grid (ceil(T / 8)), rows <= 16; all block 256
 *   reference-named fp32 DeltaNet prefill of one sequence (core.hip:5925, 6053, 6111; prefill_chunk.cpp:604-645),
 *   same parameters and grids, chunked (16 tokens) on fp32 matrix cores:
 *     halo_gdn_prefill_split(q, k, v, alpha, beta, a, dt, state, out, num_k_heads, tokens, qk_stride, v_stride,
 *       o_stride)                                                       grid (2, heads), block 256
 *     halo_gdn_chunk_prep(q, k, alpha, beta, a, dt, prep, num_k_heads, tokens, qk_stride)
 *       grid (ceil(tokens / 16), heads), block 256; prep [heads][chunks][544] floats (the engine allocates 576)
 *     halo_gdn_chunk_scan(q, k, v, prep, state, out, num_k_heads, tokens, qk_stride, v_stride, o_stride)
 *                                                                       grid (2, heads), block 256
 *   halo_shexp_down_add(dq, dd, hin, sgate, out, rows, cols, qstride)  grid ceil(rows / 32)       core.hip:2938
 *   halo_router_topk_w_y(logits, ids, weights, n, k, lstride)          grid (1, B)       batch_decode.hip:1157
 *   halo_attention_select_b_y(q, tab, tstride, kslot, gate, visible, out, scores, params, num_heads, num_kv_heads,
 *     hd, max_n, q_stride, visible_stride, scores_stride, pstride)  grid (heads, B)    batch_decode.hip:1727
 *   halo_conv_l2norm_y(in, tab, tstride, tslot, w, out, channels, kern, l2_channels, eps, stride)
 *                                                                   grid (channels / 128, B)   batch_decode.hip:1741
 *   session-union experts (batch_decode.hip:415-446, 646-697):
 *     halo_moe_bucket_b(ids, n, ucount, uexp, unum, upair)              1 block of 128; n <= 128
 *     halo_moe_down_q8r_r4_b{1..8}(qs, d, ucount, uexp, unum, upair, h, part, rows, cols, qstride)
 *                                                                       grid (ceil(rows / 32), n)
 *   prefill pair grouping (core.hip:4725-4864): halo_moe_bucket(ids, pairs, experts, sorted, pos, tiles, ntiles)
 *     1 block of 1024; halo_moe_bucket_count(ids, pairs, experts, counts) grid (chunks of 1024), block 1024;
 *     halo_moe_bucket_scan(counts, chunks, experts, tiles, ntiles, base) 1 block of 1024;
 *     halo_moe_bucket_scatter(ids, pairs, experts, chunk_off, base, sorted, pos) grid (chunks), block 1024
 *   reference-named prefill int8 GEMMs (core.hip:3103-3153, 3303-3311, 3466-3476), y [T][rows]; cols % 64 == 0:
 *     halo_gemm_q8r_wmma / _wmma_t(qs, d, xq, xd, y, rows, cols, qstride, tokens)   x as halo_quantize_q8_rows
 *       grid (ceil(T / 64), ceil(rows / 64)), block 128 / (ceil(T / 128), ceil(rows / 128)), block 256
 *     halo_gemm_q8a8_{128x128, 128x64, 320x64, 160x64, 256x128}(same)    x K-blocked (halo_quantize_q8_kblocked)
 *       grid (ceil(T / BN), ceil(rows / BM)), block 256
 *   halo_synth_q8(qs, d, rows, cols, qstride, u64 seed, f32 sigma), halo_synth_f32(x, u64 n, u64 seed, f32 sigma)
 *                                                                                              new (synthetic data)
 *   halo_stream_read(src, u64 n16, sink), halo_stream_copy(src, dst, u64 n16)   bandwidth yardsticks, new
 *   halo_clock_stamp(u64* out, u32 slot)   grid (1), block 64: out[slot] = wall clock     new (timing)
 */
#ifndef HALO_KERNELS_H_
#define HALO_KERNELS_H_

/* X(name) for every kernel the host layer launches; tests check each is present in the code object. */
#define HALO_KERNEL_LIST(X)                                                                                  \
  X(halo_repack_q8_0)                                                                                        \
  X(halo_quantize_q8_rows) X(halo_quantize_q8_rows8) X(halo_quantize_q8_rows2)                                                         \
  X(halo_q8x_cols)                                                                                           \
  X(halo_gemv_q8r) X(halo_gemv_q8r_r2) X(halo_gemv_q8r_r4)                                                   \
  X(halo_gemv_q8r_i8_r1_b1) X(halo_gemv_q8r_i8_r2_b1) X(halo_gemv_q8r_i8_r4_b1)                              \
  X(halo_gemv_q8r_i8_r4_b4) X(halo_gemv_q8r_i8x_r4_b4) X(halo_gemv_q8r_i8_r4_b8)                             \
  X(halo_gemv_q8r_i8_dual_r4_b1) X(halo_gemv_q8r_i8x_dual_r4_b4) X(halo_gemv_q8r_dual)                        \
  X(halo_gemv_q8a8_l64_r1_b1) X(halo_gemv_q8a8s_l64_r1_b1) X(halo_gemv_q8a8_l32_r1_b1) X(halo_gemv_q8a8_l16_r1_b1) \
  X(halo_gemv_q8a8_l64_r2_b4) X(halo_gemv_q8a8_l64_r2_b8)                                                    \
  X(halo_q8_half_dots)                                                                                       \
  X(halo_rmsnorm) X(halo_l2norm) X(halo_rope_neox) X(halo_rope_neox_rows) X(halo_rope_neox_p)               \
  X(halo_add) X(halo_axpy) X(halo_silu_mul) X(halo_sigmoid_gate) X(halo_copy) X(halo_copy_at)                 \
  X(halo_split_qgate) X(halo_conv_step) X(halo_conv_l2norm) X(halo_gdn_step) X(halo_gdn_step_d128)            \
  X(halo_gdn_step_d128_norm) X(halo_gated_norm) X(halo_attention_decode) X(halo_attention_prefill)           \
  X(halo_gemv_q8r_wide) X(halo_gemv_q8r_r4n) X(halo_gemv_q8r_expert) X(halo_gemv_q8r_expert_r4)             \
  X(halo_moe_down_q8r) X(halo_moe_down_q8r_r4) X(halo_moe_combine) X(halo_moe_combine_u)                      \
  X(halo_matvec_f32_rowblock) X(halo_matvec_f32_rowblock_u) X(halo_matvec_f32_rowblock2)                     \
  X(halo_matvec_f32_rowblock2_u) X(halo_quantize_q8_kblocked) X(halo_router_topk_w)                          \
  X(halo_attention_select) X(halo_attention_select_b) X(halo_attention_select_rows)                           \
  X(halo_gdn_step_d128_norm_r) X(halo_gdn_prefill_d128_norm) X(halo_conv_l2norm_prefill)                      \
  X(halo_conv_state_advance) X(halo_conv_l2norm_prefill8) X(halo_shexp_gate_up) X(halo_shexp_gate_up_u) X(halo_shexp_down_combine)         \
  X(halo_shexp_down_combine_u) X(halo_router_rowblock_q8act)                                                  \
  X(halo_moe_bucket_b) X(halo_moe_down_q8r_r4_b1) X(halo_moe_down_q8r_r4_b4) X(halo_moe_down_q8r_r4_b8)         \
  X(halo_split_qgate_norm_rope) X(halo_norm_rope_rows) X(halo_rope_neox_blocks) X(halo_rmsnorm_rows)           \
  X(halo_split_qgate_y) X(halo_rmsnorm_y) X(halo_rope_neox_p_y) X(halo_copy_at_y) X(halo_axpy_slot)            \
  X(halo_axpy_sigmoid) X(halo_axpy_sigmoid_rows) X(halo_scale_silu)                                            \
  X(halo_gemm_f32_tiled) X(halo_gemm_f32_rows) X(halo_gemm_f32_narrow) X(halo_gemm_f32_skinny)              \
  X(halo_shexp_down_add) X(halo_router_topk_w_y) X(halo_attention_select_b_y) X(halo_conv_l2norm_y)          \
  X(halo_moe_bucket) X(halo_moe_bucket_count) X(halo_moe_bucket_scan) X(halo_moe_bucket_scatter)               \
  X(halo_gemm_q8r_wmma) X(halo_gemm_q8r_wmma_t) X(halo_gemm_q8a8_128x128) X(halo_gemm_q8a8_128x64)           \
  X(halo_gemm_q8a8_320x64) X(halo_gemm_q8a8_160x64) X(halo_gemm_q8a8_256x128)                                 \
  X(halo_synth_q8) X(halo_synth_f32) X(halo_code_object_info_copy)                                            \
  X(halo_stream_read) X(halo_stream_copy) X(halo_clock_stamp)                                                 \
  X(halo_gdn_prefill_split) X(halo_gdn_chunk_prep) X(halo_gdn_chunk_scan)                                    \
  X(halo_proj_q8m_c1) X(halo_proj_q8m_c2) X(halo_proj_q8m_c4)                                            \
  X(halo_gemv_q8r_r4_b1) X(halo_gemv_q8r_r4_b8_ps) X(halo_gemv_q8r_r2_b3_p) X(halo_gemv_q8r_r2_b5_s)              \
  X(halo_gemv_q8r_dual_b1) X(halo_gemv_q8r_dual_b8_ps)

/* Module-scope variable of the code object (for halo_read_global / halo_write_global):
 *   uint32 halo_code_object_info[4] = {format version, wave size, gfx target number, spare}
 * halo_code_object_info_copy(u32* out)   grid (1), block 64: out[0..3] = halo_code_object_info as kernels see it. */

#endif /* HALO_KERNELS_H_ */
