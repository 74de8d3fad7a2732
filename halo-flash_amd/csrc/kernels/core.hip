// The gfx950 code object: every kernel the device layer can look up by name.
#include "q8.hip"
#include "moe.hip"
#include "gdn.hip"
#include "gdn_ref.hip"
#include "attn.hip"
#include "model.hip"
#include "proj.hip"
#include "moe_prefill.hip"
#include "sample.hip"
#include "ref_named.hip"

#ifdef HALO_PHASE_TIMING
extern "C" __device__ unsigned long long halo_phase_timing[6][4096][8] = {};
#endif

// Module-scope variable read and written through halo_read_global / halo_write_global (the reference's
// Device::ReadGlobal / WriteGlobal): the code object's identity {format version, wave size, target, spare}.
extern "C" __device__ std::uint32_t halo_code_object_info[4] = {1u, 64u, 950u, 0u};

// out[0..3] = halo_code_object_info as a kernel sees it. grid (1), block 64.
extern "C" __global__ void halo_code_object_info_copy(std::uint32_t* out) {
  if (threadIdx.x < 4) out[threadIdx.x] = halo_code_object_info[threadIdx.x];
}
