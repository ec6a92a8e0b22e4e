// Instantiations of the persistent decode kernel for FW_NT tokens (the build
// compiles this file once per token count, in parallel).
#include "fw_decode.h"

#ifndef FW_NT
#error "compile with -DFW_NT=<tokens>"
#endif

namespace fw {
#define FW_INSTANTIATE(NT, MBH, MBI, TK) \
    template __global__ void k_moe_decode<NT, MBH, MBI, TK>(const DecodeParams*, uint32_t);
FW_DECODE_VARIANTS_FOR(FW_INSTANTIATE, FW_NT)
#if FW_NT == 1
FW_DECODE_VARIANTS_ONE_TOKEN(FW_INSTANTIATE)
#endif
#undef FW_INSTANTIATE
}  // namespace fw
