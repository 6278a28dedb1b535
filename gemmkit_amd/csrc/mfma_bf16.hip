// mfma_bf16.hip -- bf16 instantiations of the matrix-core GEMM (f32 and bf16
// output).
#include "mma_kernel.h"

namespace gk {

hipError_t launch_mma_bf16(Tile tile, const MmaArgs &args, const EpiParams &ep, hipStream_t stream) {
    if (ep.kind == EpiKind::F32) return launch_tile<InType::BF16, EpiKind::F32>(tile, args, ep, stream);
    if (ep.kind == EpiKind::BF16) return launch_tile<InType::BF16, EpiKind::BF16>(tile, args, ep, stream);
    return hipErrorInvalidValue;
}

}  // namespace gk
