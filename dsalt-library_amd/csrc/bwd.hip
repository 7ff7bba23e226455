// Sparse-attention backward for gfx950 (placeholder until the kernels land).
#include "common.h"
#include "launch.h"

namespace dsalt {

int64_t bwd_workspace_bytes(int total_len, int num_seqs, int n_heads, int head_dim, int k_lmk) {
    (void)total_len; (void)num_seqs; (void)n_heads; (void)head_dim; (void)k_lmk;
    return 0;
}

hipError_t launch_bwd(const dsalt_bwd_args &a, hipStream_t stream) {
    (void)a; (void)stream;
    return hipErrorNotSupported;
}

}  // namespace dsalt
