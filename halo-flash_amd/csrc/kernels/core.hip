// The gfx950 code object: every kernel the device layer can look up by name.
#include "q8.hip"
#include "moe.hip"
#include "gdn.hip"
#include "attn.hip"
#include "model.hip"
#include "proj.hip"
#include "moe_prefill.hip"
#include "sample.hip"
