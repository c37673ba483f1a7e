// Prefill GEMM for GGML_OP_MUL_MAT with N > 8 activation columns, gfx950.
//
// Replaces mm_tile (crates/kernels/src/cuda/native/mm.cu:50-103). This file
// currently routes every 8-column slab through the GEMV kernels (exact int32
// block sums, f32 scaling), which is correct for any N.
#include "kernels.hpp"

namespace tlh {

tlh_status launch_gemm(const MatmulArgs &a, hipStream_t stream) {
    for (int64_t c = 0; c < a.N; c += 8) {
        MatmulArgs s = a;
        s.n0 = a.n0 + c;
        s.N = a.N - c < 8 ? a.N - c : 8;
        const tlh_status st = launch_gemv(s, nullptr, 0, stream);
        if (st != TLH_OK) return st;
    }
    return TLH_OK;
}

}  // namespace tlh
