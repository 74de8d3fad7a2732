/* Kernels of the embedded gfx950 code object (halo_core_code_object), looked up by name with halo_kernel().
 *
 * Reference-named kernels keep the reference's parameter lists and grid conventions (src/kernels/core.hip,
 * src/kernels/batch_decode.hip) so that host code launching them by name is a drop-in; the MI355X kernels under
 * new names carry their own grid conventions, documented at their definitions. Every pointer is a device buffer,
 * every other parameter a by-value scalar (src/rt/device.hpp:8-11).
 *
 *   halo_repack_q8_0(const u8* raw, i8* qs, u16* d, u32 rows, u32 cols, u32 qstride)         core.hip:2126
 *   halo_quantize_q8_rows(const f32* x, i8* xq, f32* xd, u32 cols)            grid (T)        core.hip:3089
 *   halo_q8x_cols(const f32* x, u32 xstride, u32 cols, i8* xq, f32* xs, i8* xq2, f32* xs2)   batch_decode.hip:201
 *   halo_gemv_q8r{,_r2,_r4}(const i8* qs, const u16* d, const f32* x, f32* y, u32 rows, u32 cols, u32 qstride)
 *                                                       grid ceil(rows / (8 R))              core.hip:2175,2429
 *   halo_gemv_q8r_i8{,x}_r{1,2,4}_b{1..8}(qs, d, xq, xs, xq2, xs2, y, rows, cols, qstride, ystride, groups, chunk)
 *                                                       grid (ceil(rows/(8R)) * groups, parts) batch_decode.hip:301
 *   halo_gemv_q8a8_l{16,32,64}_r{1,2,4}_b{1,2,4,8}(qs, d, xq, xs, y, rows, cols, qstride, ystride)   new (MI355X)
 *   halo_q8_half_dots(qs, xq, i32* isum, rows, cols, qstride)                                  new (parity)
 *   halo_synth_q8(qs, d, rows, cols, qstride, u64 seed, f32 sigma), halo_synth_f32(x, u64 n, u64 seed, f32 sigma)
 *                                                                                              new (synthetic data)
 */
#ifndef HALO_KERNELS_H_
#define HALO_KERNELS_H_

/* X(name) for every kernel the host layer launches; tests check each is present in the code object. */
#define HALO_KERNEL_LIST(X)                                                                                  \
  X(halo_repack_q8_0)                                                                                        \
  X(halo_quantize_q8_rows)                                                                                   \
  X(halo_q8x_cols)                                                                                           \
  X(halo_gemv_q8r) X(halo_gemv_q8r_r2) X(halo_gemv_q8r_r4)                                                   \
  X(halo_gemv_q8r_i8_r1_b1) X(halo_gemv_q8r_i8_r2_b1) X(halo_gemv_q8r_i8_r4_b1)                              \
  X(halo_gemv_q8r_i8_r4_b4) X(halo_gemv_q8r_i8x_r4_b4) X(halo_gemv_q8r_i8_r4_b8)                             \
  X(halo_gemv_q8a8_l64_r1_b1) X(halo_gemv_q8a8_l32_r1_b1) X(halo_gemv_q8a8_l16_r1_b1)                        \
  X(halo_gemv_q8a8_l64_r2_b4) X(halo_gemv_q8a8_l64_r2_b8)                                                    \
  X(halo_q8_half_dots)                                                                                       \
  X(halo_synth_q8) X(halo_synth_f32)

#endif /* HALO_KERNELS_H_ */
