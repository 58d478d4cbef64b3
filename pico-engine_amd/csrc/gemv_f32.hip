// F32 (unquantized) instantiations of the decode GEMV and small-M GEMM templates.
#include "gemv_impl.h"

namespace pe {
int gemv_f32(const GemvArgs& a, bool norm, int mode, hipStream_t s) {
    return gemv_dispatch<PE_TYPE_F32>(a, norm, mode, s);
}
int gemm_f32w(const GemmArgs& a, hipStream_t s) { return launch_qgemm<PE_TYPE_F32>(a, s); }
}  // namespace pe
