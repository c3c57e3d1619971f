// GEMM launchers (every epilogue mode) for the 256x256 tiles (batch 16).
#include "gemm_impl.h"

namespace wx {

WX_GEMM_LAUNCH_DECL(T256w8, false)
WX_GEMM_LAUNCH_DECL(T256w8, true)
WX_GEMM_LAUNCH_DECL(T256w8a3, false)

}  // namespace wx
