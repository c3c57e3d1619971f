// GEMM launchers (every epilogue mode) for the 128x128 tiles with 8 waves and a 3-slot ring.
#include "gemm_impl.h"

namespace wx {

WX_GEMM_LAUNCH_DECL(T128w8s3, false)
WX_GEMM_LAUNCH_DECL(T128w8s3, true)
WX_GEMM_LAUNCH_DECL(T128w8s3w4, false)

}  // namespace wx
