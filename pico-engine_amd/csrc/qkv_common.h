// The QKV epilogue shared by the decode QKV kernels (qkv.hip, qkv_mfma.hip): rotate-half RoPE
// of a pair of rows and the q / cache stores (model.py:175-193, rope kernels.py:37-59).
#pragma once

#include "pe_common.h"

namespace pe {

// Epilogue of a pair of rows (i, i + hd/2) of head `head` (y = W h + b): RoPE(q) into q_out,
// RoPE(k) and v into the caches at the position. An invalid position leaves the caches
// untouched and stores NaN into q.
template <int SEG>
PE_DEV void qkv_store(const pe_qkv_args& a, int64_t head, int i, float y1, float y2, float c,
                      float sn, bool pos_ok, int64_t pos) {
    const int hd = a.head_dim, half = hd / 2;
    if (SEG == 2) {
        if (pos_ok) {
            float* dst = a.v_cache + (head * a.capacity + pos) * hd;
            dst[i] = y1;
            dst[i + half] = y2;
        }
        return;
    }
    float o1 = __uint_as_float(0x7FC00000u), o2 = o1;
    if (pos_ok) {
        o1 = y1 * c - y2 * sn;
        o2 = y1 * sn + y2 * c;
    }
    if (SEG == 0) {
        const int64_t r1 = head * hd + i;
        a.q_out[r1] = o1;
        a.q_out[r1 + half] = o2;
    } else if (pos_ok) {
        float* dst = a.k_cache + (head * a.capacity + pos) * hd;
        dst[i] = o1;
        dst[i + half] = o2;
    }
}

}  // namespace pe
