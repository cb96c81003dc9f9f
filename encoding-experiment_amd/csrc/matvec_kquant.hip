// Matvec dispatch for the K-quant formats: Q4_K and the Q4_KF forms to the matrix-core
// kernel of matvec_q4k_mfma.hip, Q6_K to that of matvec_q6k_mfma.hip.
//
//   Q4_K: LC/src/cpu/ops/q4k_matvec.rs:31-90, backend.rs:126-130.
//   Q6_K (210-byte layout): LC/src/cpu/ops/q6k_matvec.rs:31-90, backend.rs:133-137.
#include "matvec_common.h"

namespace larql {

void launch_mv(const DevWeight& w, MvArgs a, hipStream_t s) {
    if (w.format == LARQL_Q4_K || w.format == LARQL_Q4_KF) return launch_q4k_mfma(w, a, s);
    if (w.format != LARQL_Q6_K) fail(LARQL_HIP_ERR_UNSUPPORTED, "launch_mv: format");
    launch_q6k_mfma(w, a, s);
}

void launch_q4k_matvec(const DevWeight& w, const float* x, float* out, size_t m, void* ws, hipStream_t s) {
    if (m > 1) {  // prefill: m tokens on the matrix cores (148-byte Q4_K)
        if (w.format != LARQL_Q4_K) fail(LARQL_HIP_ERR_UNSUPPORTED, "q4k matmul: Q4_K weights only");
        return launch_q4k_gemm(w, x, out, m, ws, s);
    }
    MvArgs a;
    a.x = x;
    a.out = out;
    launch_mv(w, a, s);
}

void launch_q6k_matvec(const DevWeight& w, const float* x, float* out, size_t m, hipStream_t s) {
    if (m != 1) fail(LARQL_HIP_ERR_UNSUPPORTED, "q6k_matvec: batch > 1 not supported");
    MvArgs a;
    a.x = x;
    a.out = out;
    launch_mv(w, a, s);
}

}  // namespace larql
