// Accessor for the embedded gfx950 code object (embed.S).
#include "halo_rt.h"

extern "C" const std::uint8_t halo_core_hsaco_begin[];
extern "C" const std::uint8_t halo_core_hsaco_end[];

extern "C" const uint8_t* halo_core_code_object(size_t* bytes) {
  if (bytes) *bytes = static_cast<size_t>(halo_core_hsaco_end - halo_core_hsaco_begin);
  return halo_core_hsaco_begin;
}
