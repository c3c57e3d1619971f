// GEMM launchers (every epilogue mode) for the 128x128 tiles with 4 waves and 128x192 tiles.
#include "gemm_impl.h"

namespace wx {

WX_GEMM_LAUNCH_DECL(T128, false)
WX_GEMM_LAUNCH_DECL(T128, true)
WX_GEMM_LAUNCH_DECL(T128x192, false)

}  // namespace wx
