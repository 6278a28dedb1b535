// mfma_i8.hip -- int8 instantiations of the matrix-core GEMM (i32 and
// requantized i8/u8 output).
#include "mma_kernel.h"

namespace gk {

hipError_t launch_mma_i8(Tile tile, const MmaArgs &args, const EpiParams &ep, hipStream_t stream) {
    if (ep.kind == EpiKind::I32) return launch_tile<InType::I8, EpiKind::I32>(tile, args, ep, stream);
    if (ep.kind == EpiKind::Q8) return launch_tile<InType::I8, EpiKind::Q8>(tile, args, ep, stream);
    return hipErrorInvalidValue;
}

}  // namespace gk
