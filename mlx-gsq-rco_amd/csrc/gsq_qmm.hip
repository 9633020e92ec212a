// QMM dispatch by type; the kernels are in gsq_qmm_impl.h, instantiated per type in
// gsq_qmm_<type>.hip.
#include <cstdio>
#include <cstdlib>

#include "gsq_common.h"

namespace gsq {

// GSQ_QMM_TUNING="mf,min_cols,waves,small_max_m,small_waves,small_nb,small_min_cols,order" (a
// prefix may be given; 0 keeps a field's default) overrides the launch plans, read once at
// library load, for measuring plans without a rebuild.
static QmmTuning qmm_tuning_from_env() {
  QmmTuning t = {0, 0, 0, 0, 0, 0, 0, 0};
  if (const char* s = std::getenv("GSQ_QMM_TUNING")) {
    int v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    std::sscanf(s, "%d,%d,%d,%d,%d,%d,%d,%d", &v[0], &v[1], &v[2], &v[3], &v[4], &v[5], &v[6], &v[7]);
    t = {v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]};
  }
  return t;
}
QmmTuning g_qmm_tuning = qmm_tuning_from_env();

hipError_t launch_qmm_q2_k(const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int64_t M,
    int64_t N, int K, const DevTables& tb, int num_cus, const QmmWorkspace& ws, hipStream_t s);
hipError_t launch_qmm_q4_k(const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int64_t M,
    int64_t N, int K, const DevTables& tb, int num_cus, const QmmWorkspace& ws, hipStream_t s);
hipError_t launch_qmm_q6_k(const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int64_t M,
    int64_t N, int K, const DevTables& tb, int num_cus, const QmmWorkspace& ws, hipStream_t s);
hipError_t launch_qmm_iq4_xs(const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int64_t M,
    int64_t N, int K, const DevTables& tb, int num_cus, const QmmWorkspace& ws, hipStream_t s);
hipError_t launch_qmm_iq3_s(const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int64_t M,
    int64_t N, int K, const DevTables& tb, int num_cus, const QmmWorkspace& ws, hipStream_t s);
hipError_t launch_qmm_iq3_xxs(const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int64_t M,
    int64_t N, int K, const DevTables& tb, int num_cus, const QmmWorkspace& ws, hipStream_t s);
hipError_t launch_qmm_iq2_xxs(const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int64_t M,
    int64_t N, int K, const DevTables& tb, int num_cus, const QmmWorkspace& ws, hipStream_t s);
hipError_t launch_qmm_iq2_xs(const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int64_t M,
    int64_t N, int K, const DevTables& tb, int num_cus, const QmmWorkspace& ws, hipStream_t s);
hipError_t launch_qmm_iq2_s(const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int64_t M,
    int64_t N, int K, const DevTables& tb, int num_cus, const QmmWorkspace& ws, hipStream_t s);
hipError_t launch_qmm_iq1_s(const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int64_t M,
    int64_t N, int K, const DevTables& tb, int num_cus, const QmmWorkspace& ws, hipStream_t s);
hipError_t launch_qmm_iq1_m(const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int64_t M,
    int64_t N, int K, const DevTables& tb, int num_cus, const QmmWorkspace& ws, hipStream_t s);

hipError_t launch_qmm(int qt, const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int64_t M, int64_t N,
                      int K, const DevTables& tb, int num_cus, const QmmWorkspace& ws, hipStream_t s) {
  switch (qt) {
    case Q2_K: return launch_qmm_q2_k(packed, x, xdt, y, ydt, M, N, K, tb, num_cus, ws, s);
    case Q4_K: return launch_qmm_q4_k(packed, x, xdt, y, ydt, M, N, K, tb, num_cus, ws, s);
    case Q6_K: return launch_qmm_q6_k(packed, x, xdt, y, ydt, M, N, K, tb, num_cus, ws, s);
    case IQ4_XS: return launch_qmm_iq4_xs(packed, x, xdt, y, ydt, M, N, K, tb, num_cus, ws, s);
    case IQ3_S: return launch_qmm_iq3_s(packed, x, xdt, y, ydt, M, N, K, tb, num_cus, ws, s);
    case IQ3_XXS: return launch_qmm_iq3_xxs(packed, x, xdt, y, ydt, M, N, K, tb, num_cus, ws, s);
    case IQ2_XXS: return launch_qmm_iq2_xxs(packed, x, xdt, y, ydt, M, N, K, tb, num_cus, ws, s);
    case IQ2_XS: return launch_qmm_iq2_xs(packed, x, xdt, y, ydt, M, N, K, tb, num_cus, ws, s);
    case IQ2_S: return launch_qmm_iq2_s(packed, x, xdt, y, ydt, M, N, K, tb, num_cus, ws, s);
    case IQ1_S: return launch_qmm_iq1_s(packed, x, xdt, y, ydt, M, N, K, tb, num_cus, ws, s);
    case IQ1_M: return launch_qmm_iq1_m(packed, x, xdt, y, ydt, M, N, K, tb, num_cus, ws, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gsq
