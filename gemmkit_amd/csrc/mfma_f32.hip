// mfma_f32.hip -- f32 instantiations of the matrix-core GEMM, and the
// per-type dispatch of launch_mma.
#include "mma_kernel.h"

namespace gk {

hipError_t launch_mma(InType in, Tile tile, const MmaArgs &args, const EpiParams &ep,
                      hipStream_t stream) {
    switch (in) {
    case InType::I8: return launch_mma_i8(tile, args, ep, stream);
    case InType::BF16: return launch_mma_bf16(tile, args, ep, stream);
    case InType::F32:
        if (ep.kind == EpiKind::F32) return launch_tile<InType::F32, EpiKind::F32>(tile, args, ep, stream);
        break;
    }
    return hipErrorInvalidValue;
}

}  // namespace gk
