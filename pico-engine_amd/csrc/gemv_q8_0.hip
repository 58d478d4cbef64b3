// Q8_0 instantiations of the dequant-GEMV (decode) and small-M GEMM (prefill) templates.
#include "gemv_impl.h"

namespace pe {
int gemv_q8_0(const GemvArgs& a, bool norm, int mode, hipStream_t s) {
    return gemv_dispatch<PE_TYPE_Q8_0>(a, norm, mode, s);
}
int gemm_q8_0(const GemmArgs& a, hipStream_t s) { return launch_qgemm<PE_TYPE_Q8_0>(a, s); }
}  // namespace pe
