// QMM kernels of IQ4_XS (one translation unit per type keeps the build parallel).
#include "gsq_qmm_impl.h"

namespace gsq {
hipError_t launch_qmm_iq4_xs(const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int64_t M, int64_t N,
                        int K, const DevTables& tb, int num_cus, const QmmWorkspace& ws, hipStream_t s) {
  return launch_qmm_type<IQ4_XS>(packed, x, xdt, y, ydt, M, N, K, tb, num_cus, ws, s);
}
}  // namespace gsq
