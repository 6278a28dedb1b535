// mfma_f32.hip -- f32 instantiations of the matrix-core GEMM, and the
// per-type dispatch of launch_mma.
#include "mma_kernel.h"

namespace gk {

hipError_t launch_mma(InType in, Tile tile, const MmaArgs &args, const EpiParams &ep,
                      hipStream_t stream) {
    // Tile rows are addressed as unsigned 32-bit offsets from the tile's
    // first row: row strides must be non-negative (the host packs otherwise).
    if (args.lda < 0 || args.ldb < 0) return hipErrorInvalidValue;
    if (tile == Tile::T256x256w8m16) return launch_mma16(in, args, ep, stream);
    if (tile == Tile::T256x352w8m16) return launch_mma16w(in, args, ep, stream);
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
