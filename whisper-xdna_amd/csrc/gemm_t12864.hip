// GEMM launchers (every epilogue mode) for the 128x64 tiles (batch 1).
#include "gemm_impl.h"

namespace wx {

WX_GEMM_LAUNCH_DECL(T12864, false)
WX_GEMM_LAUNCH_DECL(T12864, true)
WX_GEMM_LAUNCH_DECL(T12864s, false)
WX_GEMM_LAUNCH_DECL(T12864s, true)

}  // namespace wx
