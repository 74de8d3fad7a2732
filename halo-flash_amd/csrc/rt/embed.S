/* The gfx950 code object, embedded as read-only data (reference: cmake/embed.cmake, kernels::CoreHsaco()). */
  .section .rodata.halo_core,"a",@progbits
  .p2align 12
  .globl halo_core_hsaco_begin
  .hidden halo_core_hsaco_begin
halo_core_hsaco_begin:
  .incbin HALO_HSACO_PATH
  .globl halo_core_hsaco_end
  .hidden halo_core_hsaco_end
halo_core_hsaco_end:
  .section .note.GNU-stack,"",@progbits
