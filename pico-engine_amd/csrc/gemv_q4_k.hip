// Q4_K instantiations of the dequant-GEMV (decode) and small-M GEMM (prefill) templates.
#include "gemv_impl.h"

namespace pe {
int gemv_q4_k(const GemvArgs& a, bool norm, int mode, hipStream_t s) {
    return gemv_dispatch<PE_TYPE_Q4_K>(a, norm, mode, s);
}
int gemm_q4_k(const GemmArgs& a, hipStream_t s) { return launch_qgemm<PE_TYPE_Q4_K>(a, s); }
}  // namespace pe
