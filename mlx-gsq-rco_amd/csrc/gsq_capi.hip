// C ABI of libgsq.so: validation, per-device codebook tables and kernel dispatch.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../../include/gsq.h"
#include "gsq_common.h"

namespace gsq {
hipError_t launch_dequant(int qt, const uint8_t* packed, int64_t nblocks, float* out, const DevTables& t,
                          hipStream_t s);
hipError_t launch_qmv_pre(int qt, const uint8_t* packed, const void* x, void* y, int ydt, int64_t N, int K,
                          const QmvPre& pre, const DevTables& tb, int num_cus, hipStream_t s);
hipError_t launch_qmv(int qt, const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int64_t M, int64_t N,
                      int K, const DevTables& tb, int num_cus, hipStream_t s);
hipError_t launch_stage_copy(const void* src, void* dst, int64_t bytes, hipStream_t s);
hipError_t launch_qmv_group2(int qt0, const uint8_t* p0, int64_t N0, void* y0, const DevTables& tb0, int qt1,
                             const uint8_t* p1, int64_t N1, void* y1, const DevTables& tb1, const void* x, int ydt,
                             int K, int num_cus, hipStream_t s);
hipError_t launch_qmm(int qt, const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int64_t M, int64_t N,
                      int K, const DevTables& tb, int num_cus, const QmmWorkspace& ws, hipStream_t s);
hipError_t launch_embedding(int qt, const uint8_t* packed, const void* ids, int ids64, int64_t n_ids, int64_t vocab,
                            int64_t dims, void* out, int odt, const DevTables& t, hipStream_t s);
hipError_t launch_add_rms_norm(int dt, void* x, const void* delta, const void* w, void* y, int64_t rows, int dim,
                               float eps, hipStream_t s);
hipError_t launch_swiglu(int dt, const void* gu, void* out, int64_t rows, int n, hipStream_t s);
hipError_t launch_gdn_step(int dt, const GdnArgs& a, hipStream_t s);
hipError_t launch_gdn_seq(int dt, const GdnArgs& a, hipStream_t s);
hipError_t launch_attn_decode(int dt, const AttnArgs& a, hipStream_t s);
int qmv_table_bytes(int qt);
int build_qmv_table(int qt, const uint16_t* grid16, const uint8_t* ksigns, std::vector<uint8_t>& out);
int qmm_table_bytes(int qt);
int build_qmm_table(int qt, const uint16_t* grid16, const uint8_t* ksigns, std::vector<uint8_t>& out);
}  // namespace gsq

using namespace gsq;

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

const char* type_name(int t) {
  switch (t) {
    case Q2_K: return "Q2_K"; case Q4_K: return "Q4_K"; case Q6_K: return "Q6_K";
    case IQ2_XXS: return "IQ2_XXS"; case IQ2_XS: return "IQ2_XS"; case IQ3_XXS: return "IQ3_XXS";
    case IQ1_S: return "IQ1_S"; case IQ3_S: return "IQ3_S"; case IQ2_S: return "IQ2_S";
    case IQ4_XS: return "IQ4_XS"; case IQ1_M: return "IQ1_M";
    default: return "?";
  }
}

bool is_grid_type(int t) {
  int e, c;
  grid_shape_of(t, &e, &c);
  return e > 0;
}

bool uses_ksigns(int t) { return t == IQ2_XXS || t == IQ2_XS || t == IQ3_XXS; }

// Scratch of the allocation-free QMM entry point (gsq_qmm_noalloc): arrival counters (up to
// 1024 workgroups) followed by the split-tile partials of up to 256 workgroups at 64-row
// activation tiles (2 slots x 64 KiB each); the launch plan lowers the tile height until the
// partials fit. Every call on a device shares that device's copy: counters are zero when the
// code object loads and every launch leaves them at zero.
constexpr size_t kNoAllocCounterBytes = 4096;
constexpr size_t kNoAllocPartBytes = size_t(32) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocCounterBytes + kNoAllocPartBytes];

struct DevState {
  std::map<int, uint16_t*> grids;     // per grid type
  std::map<int, uint8_t*> qmv_tbls;   // per type with a QMV LDS table image
  std::map<int, uint8_t*> qmm_tbls;   // per type with a QMM LDS table image
  uint8_t* ksigns = nullptr;
  int num_cus = 0;
  uint8_t* scratch = nullptr;         // this device's address of `scratch`
  // QMM workspaces, one per stream: launches on one stream run in order, so they may share
  // a workspace; launches on different streams may overlap and never share one
  std::map<hipStream_t, QmmWorkspace> qmm_ws;
};

// True if `s` is capturing into a HIP graph: nothing may be allocated or copied
// synchronously then.
bool capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess) return false;
  return st != hipStreamCaptureStatusNone;
}

// Upload one built table image into `tbls[qt]` (allocated on first use); caller holds g_mu.
int upload_image(std::map<int, uint8_t*>& tbls, int qt, const std::vector<uint8_t>& img) {
  uint8_t*& d = tbls[qt];
  hipError_t e;
  if (!d) {
    e = hipMalloc(&d, img.size());
    if (e != hipSuccess) { tbls.erase(qt); return fail(GSQ_E_HIP, "hipMalloc: %s", hipGetErrorString(e)); }
  }
  e = hipMemcpy(d, img.data(), img.size(), hipMemcpyHostToDevice);
  if (e != hipSuccess) return fail(GSQ_E_HIP, "hipMemcpy: %s", hipGetErrorString(e));
  return GSQ_OK;
}

// Build and upload (or refresh) the QMV and QMM LDS table images of `qt` on the current device;
// caller holds g_mu. Both images are built before either is uploaded, so a codebook that one of
// them cannot hold exactly changes nothing.
int upload_qmv_table(DevState& st, int qt, const uint16_t* grid16_host, const uint8_t* ksigns_host) {
  std::vector<uint8_t> img_v, img_m;
  const int rv = build_qmv_table(qt, grid16_host, ksigns_host, img_v);
  if (rv < 0)
    return fail(GSQ_E_VALUE, "%s codebook: a value of the QMV table (codebook entry +- 0.125) is not exact in fp16",
                type_name(qt));
  const int rm = build_qmm_table(qt, grid16_host, ksigns_host, img_m);
  if (rm < 0)
    return fail(GSQ_E_VALUE, "%s codebook: a value of the QMM table (codebook entry +- 0.125) is not exact in fp16",
                type_name(qt));
  if (rv > 0)
    if (int rc = upload_image(st.qmv_tbls, qt, img_v)) return rc;
  if (rm > 0)
    if (int rc = upload_image(st.qmm_tbls, qt, img_m)) return rc;
  return GSQ_OK;
}

std::mutex g_mu;
std::map<int, DevState> g_dev;

int current_device(int* dev) {
  hipError_t e = hipGetDevice(dev);
  if (e != hipSuccess) return fail(GSQ_E_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  return GSQ_OK;
}

// Resolve the device tables for `qt` on the current device (caller holds no lock). A fixed
// table not built yet is built here unless `s` is capturing or `may_alloc` is false
// (gsq_prepare builds them first).
int resolve(int qt, DevTables* tb, int* num_cus, hipStream_t s = nullptr, bool may_alloc = true) {
  int dev;
  if (int rc = current_device(&dev)) return rc;
  std::lock_guard<std::mutex> lk(g_mu);
  DevState& st = g_dev[dev];
  if (st.num_cus == 0) {
    hipError_t e = hipDeviceGetAttribute(&st.num_cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return fail(GSQ_E_HIP, "hipDeviceGetAttribute: %s", hipGetErrorString(e));
  }
  *num_cus = st.num_cus;
  tb->grid16 = nullptr;
  tb->ksigns = st.ksigns;
  tb->qmv_tbl = nullptr;
  tb->qmm_tbl = nullptr;
  if (is_grid_type(qt)) {
    auto it = st.grids.find(qt);
    if (it == st.grids.end())
      return fail(GSQ_E_TABLES, "codebook for %s is not set on device %d (call gsq_set_tables)", type_name(qt), dev);
    tb->grid16 = it->second;
    if (uses_ksigns(qt) && !st.ksigns)
      return fail(GSQ_E_TABLES, "ksigns table is not set on device %d", dev);
  } else if (qmv_table_bytes(qt) > 0 && !st.qmv_tbls.count(qt)) {
    // fixed tables (IQ4_XS values) are built on first use on each device
    if (capturing(s))
      return fail(GSQ_E_VALUE, "the %s table is not built on device %d and the stream is capturing: "
                  "call gsq_prepare before capture", type_name(qt), dev);
    if (!may_alloc)
      return fail(GSQ_E_VALUE, "the %s table is not built on device %d: call gsq_prepare before the "
                  "allocation-free entry point", type_name(qt), dev);
    if (int rc = upload_qmv_table(st, qt, nullptr, nullptr)) return rc;
  }
  auto tt = st.qmv_tbls.find(qt);
  if (tt != st.qmv_tbls.end()) tb->qmv_tbl = tt->second;
  auto mt = st.qmm_tbls.find(qt);
  if (mt != st.qmm_tbls.end()) tb->qmm_tbl = mt->second;
  return GSQ_OK;
}

// Partial-tile capacity of a QMM workspace: 2 slots of up to 256 x 256 floats per CU (the
// largest tile plan), and one arrival counter per CU.
long long qmm_ws_part_bytes(int num_cus) { return 2ll * num_cus * 256 * 256 * (long long)sizeof(float); }

// The QMM workspace of stream `s` on the current device, allocated on the first QMM call on
// that stream (or by gsq_prepare); counters start at zero and every launch leaves them at zero.
int qmm_workspace(hipStream_t s, QmmWorkspace* ws) {
  int dev;
  if (int rc = current_device(&dev)) return rc;
  std::lock_guard<std::mutex> lk(g_mu);
  DevState& st = g_dev[dev];
  auto it = st.qmm_ws.find(s);
  if (it != st.qmm_ws.end()) {
    *ws = it->second;
    return GSQ_OK;
  }
  if (capturing(s))
    return fail(GSQ_E_VALUE, "stream has no QMM workspace on device %d and is capturing: call gsq_prepare(stream) "
                "before capture", dev);
  if (st.qmm_ws.size() >= 64)
    return fail(GSQ_E_VALUE, "QMM workspaces exist for 64 streams on device %d; reuse streams", dev);
  if (st.num_cus == 0) {
    hipError_t e = hipDeviceGetAttribute(&st.num_cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return fail(GSQ_E_HIP, "hipDeviceGetAttribute: %s", hipGetErrorString(e));
  }
  const int groups = st.num_cus;
  const long long part_bytes = qmm_ws_part_bytes(groups);
  float* part = nullptr;
  int* cnt = nullptr;
  hipError_t e = hipMalloc(&part, (size_t)part_bytes);
  if (e != hipSuccess) return fail(GSQ_E_HIP, "hipMalloc(QMM workspace): %s", hipGetErrorString(e));
  e = hipMalloc(&cnt, (size_t)groups * sizeof(int));
  if (e == hipSuccess) e = hipMemset(cnt, 0, (size_t)groups * sizeof(int));
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    hipFree(part);
    if (cnt) hipFree(cnt);
    return fail(GSQ_E_HIP, "QMM workspace setup: %s", hipGetErrorString(e));
  }
  *ws = st.qmm_ws[s] = QmmWorkspace{part, cnt, groups, part_bytes};
  return GSQ_OK;
}

// This device's address of `scratch` (host code never passes the symbol itself: on the host it
// names a shadow variable, not device memory); looked up once per device, with it current.
int noalloc_scratch(uint8_t** p, int* num_cus) {
  int dev;
  if (int rc = current_device(&dev)) return rc;
  std::lock_guard<std::mutex> lk(g_mu);
  DevState& st = g_dev[dev];
  if (st.num_cus == 0) {
    hipError_t e = hipDeviceGetAttribute(&st.num_cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return fail(GSQ_E_HIP, "hipDeviceGetAttribute: %s", hipGetErrorString(e));
  }
  if (!st.scratch) {
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(GSQ_E_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    st.scratch = static_cast<uint8_t*>(ptr);
  }
  *p = st.scratch;
  *num_cus = st.num_cus;
  return GSQ_OK;
}

// True if the byte ranges [a, a + an) and [b, b + bn) share a byte (a NULL range shares none).
bool overlaps(const void* a, int64_t an, const void* b, int64_t bn) {
  if (!a || !b) return false;
  const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
  return pa < pb + (uintptr_t)bn && pb < pa + (uintptr_t)an;
}

int check_common(int qt, const void* packed, int64_t M, int64_t N, int64_t K, int xdt, int ydt) {
  if (block_bytes_of(qt) == 0) return fail(GSQ_E_UNSUPPORTED, "unsupported quant type id %d", qt);
  if (K <= 0 || K % 256) return fail(GSQ_E_VALUE, "invalid %s matrix width %lld", type_name(qt), (long long)K);
  if (N <= 0 || M <= 0) return fail(GSQ_E_VALUE, "invalid shape M=%lld N=%lld", (long long)M, (long long)N);
  if (K > (1ll << 30) || N > (1ll << 40)) return fail(GSQ_E_VALUE, "matrix too large");
  if (!packed) return fail(GSQ_E_VALUE, "packed is NULL");
  if (reinterpret_cast<uintptr_t>(packed) & 1) return fail(GSQ_E_VALUE, "packed must be 2-byte aligned");
  if (xdt < 0 || xdt > 2 || ydt < 0 || ydt > 2) return fail(GSQ_E_TYPE, "bad dtype code x=%d y=%d", xdt, ydt);
  return GSQ_OK;
}

}  // namespace

extern "C" {

int gsq_version(void) { return 1; }

int gsq_block_bytes(int qtype_id) {
  int bb = block_bytes_of(qtype_id);
  return bb ? bb : -1;
}

const char* gsq_last_error(void) { return g_err.c_str(); }

int gsq_set_tables(int qt, const float* grid, int64_t entries, int64_t coords, const uint8_t* ksigns,
                   int64_t n_ksigns) {
  if (block_bytes_of(qt) == 0) return fail(GSQ_E_UNSUPPORTED, "unsupported quant type id %d", qt);
  int ee, cc;
  grid_shape_of(qt, &ee, &cc);
  if (ee == 0) return fail(GSQ_E_VALUE, "%s has no codebook", type_name(qt));
  if (!grid || entries != ee || coords != cc)
    return fail(GSQ_E_VALUE, "%s codebook must be %dx%d, got %lldx%lld", type_name(qt), ee, cc,
                (long long)entries, (long long)coords);
  if (!ksigns || n_ksigns != 128) return fail(GSQ_E_VALUE, "ksigns must have 128 entries");
  // the QMV decoders form the sign byte from the table's closed form (every published ksigns
  // table has it); a different table would make them disagree with the other kernels
  for (int i = 0; i < 128; ++i)
    if (ksigns[i] != (uint8_t)(i | ((__builtin_popcount((unsigned)i) & 1) << 7)))
      return fail(GSQ_E_VALUE, "ksigns[%d] is %d: the table must be the published one (entry i = i with bit 7 "
                  "the parity of i)", i, (int)ksigns[i]);
  std::vector<uint16_t> h16((size_t)ee * cc);
  for (size_t i = 0; i < h16.size(); ++i) {
    const float v = grid[i];
    const _Float16 h = (_Float16)v;
    if (!std::isfinite(v) || (float)h != v)
      return fail(GSQ_E_VALUE, "%s codebook value %g at %zu is not exact in fp16", type_name(qt), (double)v, i);
    h16[i] = __builtin_bit_cast(uint16_t, h);
  }
  {  // the table images must hold the codebook exactly (IQ1's hold entry +- 0.125): check first
    std::vector<uint8_t> img;
    if (build_qmv_table(qt, h16.data(), ksigns, img) < 0 || build_qmm_table(qt, h16.data(), ksigns, img) < 0)
      return fail(GSQ_E_VALUE, "%s codebook: entry +- 0.125 is not exact in fp16 for some value", type_name(qt));
  }
  int dev;
  if (int rc = current_device(&dev)) return rc;
  std::lock_guard<std::mutex> lk(g_mu);
  DevState& st = g_dev[dev];
  hipError_t e;
  if (!st.ksigns) {
    e = hipMalloc(&st.ksigns, 128);
    if (e != hipSuccess) { st.ksigns = nullptr; return fail(GSQ_E_HIP, "hipMalloc: %s", hipGetErrorString(e)); }
  }
  e = hipMemcpy(st.ksigns, ksigns, 128, hipMemcpyHostToDevice);
  if (e != hipSuccess) return fail(GSQ_E_HIP, "hipMemcpy: %s", hipGetErrorString(e));
  uint16_t*& g = st.grids[qt];
  if (!g) {
    e = hipMalloc(&g, h16.size() * 2);
    if (e != hipSuccess) { st.grids.erase(qt); return fail(GSQ_E_HIP, "hipMalloc: %s", hipGetErrorString(e)); }
  }
  e = hipMemcpy(g, h16.data(), h16.size() * 2, hipMemcpyHostToDevice);
  if (e != hipSuccess) return fail(GSQ_E_HIP, "hipMemcpy: %s", hipGetErrorString(e));
  // the QMV and QMM table images of every type that reads this codebook or the ksigns table
  for (int t : {IQ1_S, IQ1_M, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S}) {
    if (t != qt && !(uses_ksigns(t) && st.qmv_tbls.count(t))) continue;
    auto git = st.grids.find(t);
    if (git == st.grids.end()) continue;
    std::vector<uint16_t> gh;
    if (t == qt) gh = h16;
    else {
      int te, tc;
      grid_shape_of(t, &te, &tc);
      gh.resize((size_t)te * tc);
      e = hipMemcpy(gh.data(), git->second, gh.size() * 2, hipMemcpyDeviceToHost);
      if (e != hipSuccess) return fail(GSQ_E_HIP, "hipMemcpy: %s", hipGetErrorString(e));
    }
    if (int rc = upload_qmv_table(st, t, gh.data(), ksigns)) return rc;
  }
  return GSQ_OK;
}

int gsq_prepare(void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (capturing(s)) return fail(GSQ_E_VALUE, "gsq_prepare must be called before the stream starts capturing");
  for (int qt : {Q2_K, Q4_K, Q6_K, IQ4_XS}) {  // the types whose tables are fixed (built here)
    DevTables tb;
    int cus;
    if (int rc = resolve(qt, &tb, &cus, s)) return rc;
  }
  QmmWorkspace ws;
  if (int rc = qmm_workspace(s, &ws)) return rc;
  uint8_t* sp;
  int cus;
  return noalloc_scratch(&sp, &cus);
}

int gsq_tables_ready(int qt) {
  if (block_bytes_of(qt) == 0) return 0;
  if (!is_grid_type(qt)) return 1;
  DevTables tb;
  int cus;
  return resolve(qt, &tb, &cus) == GSQ_OK ? 1 : 0;
}

int gsq_dequant(int qt, const void* packed, int64_t nblocks, float* out, void* stream) {
  if (block_bytes_of(qt) == 0) return fail(GSQ_E_UNSUPPORTED, "unsupported quant type id %d", qt);
  if (nblocks < 0) return fail(GSQ_E_VALUE, "negative block count");
  if (nblocks == 0) return GSQ_OK;
  if (!packed || !out) return fail(GSQ_E_VALUE, "NULL pointer");
  if (reinterpret_cast<uintptr_t>(out) & 15) return fail(GSQ_E_VALUE, "out must be 16-byte aligned");
  DevTables tb;
  int cus;
  if (int rc = resolve(qt, &tb, &cus, static_cast<hipStream_t>(stream))) return rc;
  hipError_t e = launch_dequant(qt, static_cast<const uint8_t*>(packed), nblocks, out, tb,
                                static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(GSQ_E_HIP, "dequant launch: %s", hipGetErrorString(e));
  return GSQ_OK;
}

int gsq_qmv(int qt, const void* packed, const void* x, int xdt, void* y, int ydt, int64_t M, int64_t N, int64_t K,
            void* stream) {
  if (int rc = check_common(qt, packed, M, N, K, xdt, ydt)) return rc;
  if (!x || !y) return fail(GSQ_E_VALUE, "NULL pointer");
  if (K > (xdt == GSQ_F16 ? 65536 : 32768))
    return fail(GSQ_E_VALUE, "QMV supports K <= %d for this activation dtype (got %lld); use gsq_qmm",
                xdt == GSQ_F16 ? 65536 : 32768, (long long)K);
  const int64_t xe = xdt == GSQ_F32 ? 4 : 2;
  if (reinterpret_cast<uintptr_t>(x) & (xe - 1)) return fail(GSQ_E_VALUE, "x is not aligned to its element size");
  hipStream_t s = static_cast<hipStream_t>(stream);
  DevTables tb;
  int cus;
  if (int rc = resolve(qt, &tb, &cus, s)) return rc;
  const uint8_t* pk = static_cast<const uint8_t*>(packed);
  if ((reinterpret_cast<uintptr_t>(x) & 15) == 0) {
    hipError_t e = launch_qmv(qt, pk, x, xdt, y, ydt, M, N, (int)K, tb, cus, s);
    if (e != hipSuccess) return fail(GSQ_E_HIP, "qmv launch: %s", hipGetErrorString(e));
    return GSQ_OK;
  }
  // x not 16-byte aligned (the kernels read it in 16-byte pieces): rows are copied into the
  // stream's QMM workspace first, as many per launch as it holds; stream order keeps the copies
  // and the launches that read them (and any QMM launch on the stream) apart
  QmmWorkspace ws;
  if (int rc = qmm_workspace(s, &ws)) return rc;
  const int64_t row_bytes = K * xe, chunk = ws.part_bytes / row_bytes;
  if (chunk < 1) return fail(GSQ_E_VALUE, "x row of %lld bytes exceeds the staging workspace", (long long)row_bytes);
  const int64_t ye = ydt == GSQ_F32 ? 4 : 2;
  for (int64_t r = 0; r < M; r += chunk) {
    const int64_t rows = M - r < chunk ? M - r : chunk;
    hipError_t e = launch_stage_copy(static_cast<const uint8_t*>(x) + r * row_bytes, ws.part, rows * row_bytes, s);
    if (e == hipSuccess)
      e = launch_qmv(qt, pk, ws.part, xdt, static_cast<uint8_t*>(y) + r * N * ye, ydt, rows, N, (int)K, tb, cus, s);
    if (e != hipSuccess) return fail(GSQ_E_HIP, "qmv launch: %s", hipGetErrorString(e));
  }
  return GSQ_OK;
}

int gsq_qmv_group2(int qt0, const void* packed0, int64_t N0, void* y0, int qt1, const void* packed1, int64_t N1,
                   void* y1, const void* x, int y_dtype, int64_t K, void* stream) {
  if (int rc = check_common(qt0, packed0, 1, N0, K, GSQ_F16, y_dtype)) return rc;
  if (int rc = check_common(qt1, packed1, 1, N1, K, GSQ_F16, y_dtype)) return rc;
  if (!x || !y0 || !y1) return fail(GSQ_E_VALUE, "NULL pointer");
  if (K > 65536) return fail(GSQ_E_VALUE, "QMV supports K <= 65536 for fp16 activations (got %lld)", (long long)K);
  if (reinterpret_cast<uintptr_t>(x) & 1) return fail(GSQ_E_VALUE, "x is not aligned to its element size");
  // every workgroup reads x while others already write their outputs
  const int64_t ye = y_dtype == GSQ_F32 ? 4 : 2;
  if (overlaps(y0, N0 * ye, y1, N1 * ye) || overlaps(y0, N0 * ye, x, K * 2) || overlaps(y1, N1 * ye, x, K * 2))
    return fail(GSQ_E_VALUE, "y0, y1 and x must not overlap");
  hipStream_t s = static_cast<hipStream_t>(stream);
  DevTables tb0, tb1;
  int cus;
  if (int rc = resolve(qt0, &tb0, &cus, s)) return rc;
  if (int rc = resolve(qt1, &tb1, &cus, s)) return rc;
  if ((reinterpret_cast<uintptr_t>(x) & 15) == 0) {
    hipError_t e = launch_qmv_group2(qt0, static_cast<const uint8_t*>(packed0), N0, y0, tb0, qt1,
                                     static_cast<const uint8_t*>(packed1), N1, y1, tb1, x, y_dtype, (int)K, cus, s);
    if (e == hipSuccess) return GSQ_OK;
    if (e != hipErrorNotSupported) return fail(GSQ_E_HIP, "qmv group launch: %s", hipGetErrorString(e));
  }
  // (for tests of the shared kernel: refuse instead of launching the products one by one)
  if (std::getenv("GSQ_QMV_GROUP_NO_FALLBACK"))
    return fail(GSQ_E_UNSUPPORTED, "the shared kernel does not take these two products");
  // the two products one by one (plans the shared kernel does not take, or an x to stage)
  if (int rc = gsq_qmv(qt0, packed0, x, GSQ_F16, y0, y_dtype, 1, N0, K, stream)) return rc;
  return gsq_qmv(qt1, packed1, x, GSQ_F16, y1, y_dtype, 1, N1, K, stream);
}

int gsq_qmv_pre(int qt, const void* packed, int pre_op, const void* x, const void* pre_a, const void* pre_w,
                float eps, void* res_out, void* x_out, void* y, int ydt, int64_t N, int64_t K, void* conv_state,
                const void* conv_w, int64_t conv_rows, int64_t conv_kernel, float* conv_out, void* stream) {
  if (int rc = check_common(qt, packed, 1, N, K, GSQ_F16, ydt)) return rc;
  if (pre_op != GSQ_PRE_ADD_RMSNORM && pre_op != GSQ_PRE_SWIGLU) return fail(GSQ_E_VALUE, "unknown pre_op %d", pre_op);
  if (conv_rows < 0 || conv_rows > N) return fail(GSQ_E_VALUE, "conv_rows must be 0..N");
  if (conv_rows > 0) {
    if (!conv_state || !conv_w || !conv_out) return fail(GSQ_E_VALUE, "convolution pointer is NULL");
    if (conv_kernel < 2 || conv_kernel > 8) return fail(GSQ_E_VALUE, "convolution kernel must be 2..8");
    if (ydt != GSQ_F16) return fail(GSQ_E_VALUE, "the convolution epilogue needs fp16 y");
  }
  if (!x || !y) return fail(GSQ_E_VALUE, "NULL pointer");
  if (pre_op == GSQ_PRE_ADD_RMSNORM && !pre_w) return fail(GSQ_E_VALUE, "the norm weight is NULL");
  if (pre_op == GSQ_PRE_ADD_RMSNORM && !(eps >= 0.f)) return fail(GSQ_E_VALUE, "eps must be >= 0");
  if (K % 8 || K > 32768) return fail(GSQ_E_VALUE, "K must be a multiple of 8 up to 32768 (got %lld)", (long long)K);
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(pre_a) | reinterpret_cast<uintptr_t>(pre_w) |
       reinterpret_cast<uintptr_t>(res_out) | reinterpret_cast<uintptr_t>(x_out)) & 15)
    return fail(GSQ_E_VALUE, "x, pre_a, pre_w, res_out and x_out must be 16-byte aligned");
  // workgroup 0 writes res_out and x_out while the other workgroups still read x, pre_a and
  // pre_w: an output that overlaps an input (or the other output) would race
  const int64_t kb = K * 2, xb = (pre_op == GSQ_PRE_SWIGLU ? 2 : 1) * kb;
  const bool norm = pre_op == GSQ_PRE_ADD_RMSNORM;
  const void* outs[2] = {norm ? res_out : nullptr, x_out};
  const char* out_names[2] = {"res_out", "x_out"};
  for (int i = 0; i < 2; ++i) {
    if (!outs[i]) continue;
    if (overlaps(outs[i], kb, x, xb) || (norm && (overlaps(outs[i], kb, pre_a, kb) || overlaps(outs[i], kb, pre_w, kb))))
      return fail(GSQ_E_VALUE, "%s must not alias x, pre_a or pre_w (other workgroups still read them)", out_names[i]);
  }
  if (outs[0] && overlaps(outs[0], kb, outs[1], kb)) return fail(GSQ_E_VALUE, "res_out and x_out must not alias");
  QmvPre pre;
  pre.op = pre_op == GSQ_PRE_ADD_RMSNORM ? QMV_PRE_ADD_NORM : QMV_PRE_SWIGLU;
  pre.a = pre_op == GSQ_PRE_SWIGLU ? x : pre_a;
  pre.w = pre_w;
  pre.res = pre_op == GSQ_PRE_ADD_RMSNORM ? res_out : nullptr;
  pre.out = x_out;
  pre.eps = eps;
  if (conv_rows > 0) {
    pre.conv_state = conv_state;
    pre.conv_w = conv_w;
    pre.conv_out = conv_out;
    pre.conv_rows = (int)conv_rows;
    pre.conv_k = (int)conv_kernel;
  }
  DevTables tb;
  int cus;
  if (int rc = resolve(qt, &tb, &cus, static_cast<hipStream_t>(stream))) return rc;
  hipError_t e = launch_qmv_pre(qt, static_cast<const uint8_t*>(packed), x, y, ydt, N, (int)K, pre, tb, cus,
                                static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(GSQ_E_HIP, "qmv launch: %s", hipGetErrorString(e));
  return GSQ_OK;
}

int gsq_qmm(int qt, const void* packed, const void* x, int xdt, void* y, int ydt, int64_t M, int64_t N, int64_t K,
            void* stream) {
  if (int rc = check_common(qt, packed, M, N, K, xdt, ydt)) return rc;
  if (!x || !y) return fail(GSQ_E_VALUE, "NULL pointer");
  DevTables tb;
  int cus;
  if (int rc = resolve(qt, &tb, &cus, static_cast<hipStream_t>(stream))) return rc;
  QmmWorkspace ws;
  if (int rc = qmm_workspace(static_cast<hipStream_t>(stream), &ws)) return rc;
  hipError_t e = launch_qmm(qt, static_cast<const uint8_t*>(packed), x, xdt, y, ydt, M, N, (int)K, tb, cus, ws,
                            static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(GSQ_E_HIP, "qmm launch: %s", hipGetErrorString(e));
  return GSQ_OK;
}

int gsq_qmm_noalloc(int qt, const void* packed, const void* x, int xdt, void* y, int ydt, int64_t M, int64_t N,
                    int64_t K, void* stream) {
  if (int rc = check_common(qt, packed, M, N, K, xdt, ydt)) return rc;
  if (!x || !y) return fail(GSQ_E_VALUE, "NULL pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  DevTables tb;
  int cus;
  if (int rc = resolve(qt, &tb, &cus, s, /*may_alloc=*/false)) return rc;
  uint8_t* sp;
  if (int rc = noalloc_scratch(&sp, &cus)) return rc;
  // the partials of one workgroup per CU at the smallest tile plan (64-row tiles: 2 slots of
  // 64 KiB) must fit the scratch
  const long long need = 2ll * cus * 64 * 1024;
  if (cus > (int)(kNoAllocCounterBytes / sizeof(int)) || need > (long long)kNoAllocPartBytes)
    return fail(GSQ_E_VALUE, "gsq_qmm_noalloc: %d workgroups need %lld bytes of partial tiles; its scratch holds "
                "%zu (use gsq_qmm)", cus, need, kNoAllocPartBytes);
  QmmWorkspace ws{reinterpret_cast<float*>(sp + kNoAllocCounterBytes), reinterpret_cast<int*>(sp),
                  (int)(kNoAllocCounterBytes / sizeof(int)), (long long)kNoAllocPartBytes};
  hipError_t e = launch_qmm(qt, static_cast<const uint8_t*>(packed), x, xdt, y, ydt, M, N, (int)K, tb, cus, ws, s);
  if (e != hipSuccess) return fail(GSQ_E_HIP, "qmm launch: %s", hipGetErrorString(e));
  return GSQ_OK;
}

int gsq_embedding(int qt, const void* packed, const void* ids, int ids_dtype, int64_t n_ids, int64_t vocab,
                  int64_t dims, void* out, int out_dtype, void* stream) {
  if (block_bytes_of(qt) == 0) return fail(GSQ_E_UNSUPPORTED, "unsupported quant type id %d", qt);
  if (ids_dtype != GSQ_IDS_I32 && ids_dtype != GSQ_IDS_I64) return fail(GSQ_E_TYPE, "ids must be int32 or int64");
  if (out_dtype != GSQ_F32 && out_dtype != GSQ_F16 && out_dtype != GSQ_BF16)
    return fail(GSQ_E_TYPE, "unsupported output dtype code %d", out_dtype);
  if (dims <= 0 || dims % 256) return fail(GSQ_E_VALUE, "embedding dimensions must be divisible by 256");
  if (n_ids < 0 || vocab < 0) return fail(GSQ_E_VALUE, "negative id count or vocabulary size");
  if (n_ids == 0) return GSQ_OK;
  if (!packed || !ids || !out) return fail(GSQ_E_VALUE, "NULL pointer");
  if (reinterpret_cast<uintptr_t>(out) & 15) return fail(GSQ_E_VALUE, "out must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(ids) & (ids_dtype == GSQ_IDS_I64 ? 7 : 3)) return fail(GSQ_E_VALUE, "misaligned ids");
  DevTables tb;
  int cus;
  if (int rc = resolve(qt, &tb, &cus, static_cast<hipStream_t>(stream))) return rc;
  hipError_t e = launch_embedding(qt, static_cast<const uint8_t*>(packed), ids, ids_dtype == GSQ_IDS_I64, n_ids, vocab,
                                  dims, out, out_dtype, tb, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(GSQ_E_HIP, "embedding launch: %s", hipGetErrorString(e));
  return GSQ_OK;
}

int gsq_add_rms_norm(void* x, const void* delta, const void* w, void* y, int64_t rows, int64_t dim, float eps,
                     int dtype, void* stream) {
  if (dtype != GSQ_F32 && dtype != GSQ_F16 && dtype != GSQ_BF16) return fail(GSQ_E_TYPE, "unsupported dtype code %d", dtype);
  if (rows < 0 || dim <= 0 || rows >= (1ll << 31)) return fail(GSQ_E_VALUE, "invalid shape");
  if (rows == 0) return GSQ_OK;
  if (!x || !w || !y) return fail(GSQ_E_VALUE, "NULL pointer");
  if (!(eps >= 0.f)) return fail(GSQ_E_VALUE, "eps must be >= 0");
  if (dim % 8 || dim > 8192) return fail(GSQ_E_VALUE, "row length must be a multiple of 8 up to 8192");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(delta) | reinterpret_cast<uintptr_t>(w) |
       reinterpret_cast<uintptr_t>(y)) & 15)
    return fail(GSQ_E_VALUE, "x, delta, w and y must be 16-byte aligned");
  hipError_t e = launch_add_rms_norm(dtype, x, delta, w, y, rows, (int)dim, eps, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(GSQ_E_HIP, "add_rms_norm launch: %s", hipGetErrorString(e));
  return GSQ_OK;
}

int gsq_swiglu(const void* gate_up, void* out, int64_t rows, int64_t n, int dtype, void* stream) {
  if (dtype != GSQ_F32 && dtype != GSQ_F16 && dtype != GSQ_BF16) return fail(GSQ_E_TYPE, "unsupported dtype code %d", dtype);
  if (rows < 0 || n <= 0 || n >= (1ll << 30)) return fail(GSQ_E_VALUE, "invalid shape");
  if (rows == 0) return GSQ_OK;
  if (!gate_up || !out) return fail(GSQ_E_VALUE, "NULL pointer");
  hipError_t e = launch_swiglu(dtype, gate_up, out, rows, (int)n, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(GSQ_E_HIP, "swiglu launch: %s", hipGetErrorString(e));
  return GSQ_OK;
}

int gsq_gdn_step(const void* qkv, int64_t qkv_stride, const void* z, int64_t z_stride, const void* x,
                 int64_t x_stride, const void* w_ab, int64_t hidden, void* conv_state, const void* conv_w,
                 const float* ssm_a, const float* dt_bias, float* rec_state, const void* norm_w, void* out,
                 int64_t out_stride, float* work, int64_t batch, int64_t key_heads, int64_t value_heads,
                 int64_t head_k_dim, int64_t head_v_dim, int64_t conv_kernel, float eps, int dtype, void* stream) {
  if (dtype != GSQ_F32 && dtype != GSQ_F16 && dtype != GSQ_BF16) return fail(GSQ_E_TYPE, "unsupported dtype code %d", dtype);
  if (batch < 0 || batch > 65535) return fail(GSQ_E_VALUE, "batch must be 0..65535");
  if (batch == 0) return GSQ_OK;
  if (key_heads <= 0 || value_heads <= 0 || value_heads % key_heads || value_heads > 65535)
    return fail(GSQ_E_VALUE, "value heads must be a positive multiple of key heads (at most 65535)");
  if (head_k_dim <= 0 || head_k_dim > 128 || head_k_dim % 4) return fail(GSQ_E_VALUE, "key head dim must be a multiple of 4 up to 128");
  if (head_v_dim <= 0 || head_v_dim % 64 || head_v_dim > 256) return fail(GSQ_E_VALUE, "value head dim must be 64, 128, 192 or 256");
  if (conv_kernel < 2 || conv_kernel > 8) return fail(GSQ_E_VALUE, "convolution kernel must be 2..8");
  if (hidden <= 0 || hidden >= (1ll << 30)) return fail(GSQ_E_VALUE, "invalid hidden size");
  if (!z || !x || !w_ab || !ssm_a || !dt_bias || !rec_state || !norm_w || !out || !work)
    return fail(GSQ_E_VALUE, "NULL pointer");
  if (conv_state && (!qkv || !conv_w)) return fail(GSQ_E_VALUE, "NULL pointer");
  if (!(eps >= 0.f)) return fail(GSQ_E_VALUE, "eps must be >= 0");
  GdnArgs a;
  a.qkv = qkv; a.z = z; a.x = x; a.w_ab = w_ab; a.conv = conv_state; a.conv_w = conv_w; a.ssm_a = ssm_a;
  a.dt_bias = dt_bias; a.rec = rec_state; a.norm_w = norm_w; a.out = out; a.work = work;
  a.qkv_stride = qkv_stride; a.z_stride = z_stride; a.x_stride = x_stride; a.out_stride = out_stride;
  a.B = (int)batch; a.Hk = (int)key_heads; a.Hv = (int)value_heads; a.dk = (int)head_k_dim; a.dv = (int)head_v_dim;
  a.K = (int)conv_kernel; a.hidden = (int)hidden; a.eps = eps;
  hipError_t e = launch_gdn_step(dtype, a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(GSQ_E_HIP, "gdn_step launch: %s", hipGetErrorString(e));
  return GSQ_OK;
}

int gsq_gdn_seq(const void* qkv, int64_t qkv_stride, const void* z, int64_t z_stride, const void* ab,
                int64_t ab_stride, void* conv_state, const void* conv_w, const float* ssm_a, const float* dt_bias,
                float* rec_state, const void* norm_w, void* out, int64_t out_stride, float* work, int64_t batch,
                int64_t seq, int64_t key_heads, int64_t value_heads, int64_t head_k_dim, int64_t head_v_dim,
                int64_t conv_kernel, float eps, int dtype, void* stream) {
  if (dtype != GSQ_F32 && dtype != GSQ_F16 && dtype != GSQ_BF16) return fail(GSQ_E_TYPE, "unsupported dtype code %d", dtype);
  if (batch < 0 || batch > 65535 || seq < 0 || seq > 65535) return fail(GSQ_E_VALUE, "batch and seq must be 0..65535");
  if (batch == 0 || seq == 0) return GSQ_OK;
  if (key_heads <= 0 || value_heads <= 0 || value_heads % key_heads || value_heads > 65535)
    return fail(GSQ_E_VALUE, "value heads must be a positive multiple of key heads (at most 65535)");
  if (head_k_dim <= 0 || head_k_dim > 128 || head_k_dim % 4) return fail(GSQ_E_VALUE, "key head dim must be a multiple of 4 up to 128");
  if (head_v_dim <= 0 || head_v_dim % 64 || head_v_dim > 256) return fail(GSQ_E_VALUE, "value head dim must be 64, 128, 192 or 256");
  if (conv_kernel < 2 || conv_kernel > 8) return fail(GSQ_E_VALUE, "convolution kernel must be 2..8");
  if (!qkv || !z || !ab || !conv_state || !conv_w || !ssm_a || !dt_bias || !rec_state || !norm_w || !out || !work)
    return fail(GSQ_E_VALUE, "NULL pointer");
  if (!(eps >= 0.f)) return fail(GSQ_E_VALUE, "eps must be >= 0");
  GdnArgs a;
  a.qkv = qkv; a.z = z; a.x = nullptr; a.w_ab = nullptr; a.conv = conv_state; a.conv_w = conv_w; a.ssm_a = ssm_a;
  a.dt_bias = dt_bias; a.rec = rec_state; a.norm_w = norm_w; a.out = out; a.work = work;
  a.qkv_stride = qkv_stride; a.z_stride = z_stride; a.x_stride = 0; a.out_stride = out_stride;
  a.B = (int)batch; a.Hk = (int)key_heads; a.Hv = (int)value_heads; a.dk = (int)head_k_dim; a.dv = (int)head_v_dim;
  a.K = (int)conv_kernel; a.hidden = 0; a.eps = eps;
  a.S = (int)seq; a.ab = ab; a.ab_stride = ab_stride;
  hipError_t e = launch_gdn_seq(dtype, a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(GSQ_E_HIP, "gdn_seq launch: %s", hipGetErrorString(e));
  return GSQ_OK;
}

int gsq_attn_decode(const void* qg, int64_t qg_stride, const void* k, int64_t k_stride, const void* v,
                    int64_t v_stride, const void* q_norm_w, const void* k_norm_w, const double* inv_freq,
                    void* k_cache, void* v_cache, const int64_t* pos, void* out, int64_t out_stride, int64_t batch,
                    int64_t heads, int64_t kv_heads, int64_t head_dim, int64_t rotary_dim, int64_t max_len,
                    float eps, float* work, int64_t chunk, int dtype, void* stream) {
  if (dtype != GSQ_F32 && dtype != GSQ_F16 && dtype != GSQ_BF16) return fail(GSQ_E_TYPE, "unsupported dtype code %d", dtype);
  if (batch < 0 || batch > 65535) return fail(GSQ_E_VALUE, "batch must be 0..65535");
  if (batch == 0) return GSQ_OK;
  if (kv_heads <= 0 || heads <= 0 || heads % kv_heads || heads > 65535)
    return fail(GSQ_E_VALUE, "heads must be a positive multiple of kv heads (at most 65535)");
  if (head_dim <= 0 || head_dim > 256 || head_dim % 4) return fail(GSQ_E_VALUE, "head dim must be a multiple of 4 up to 256");
  if (rotary_dim < 0 || rotary_dim > head_dim || rotary_dim % 2) return fail(GSQ_E_VALUE, "invalid rotary dim");
  if (work && (chunk < 64 || chunk > 1024 || chunk % 64))
    return fail(GSQ_E_VALUE, "chunk must be a multiple of 64 from 64 to 1024");
  if (max_len <= 0 || max_len > (work ? (1 << 20) : 32768))
    return fail(GSQ_E_VALUE, "cache length must be 1..%d", work ? (1 << 20) : 32768);
  if (!qg || !k || !v || !q_norm_w || !k_norm_w || (!inv_freq && rotary_dim) || !k_cache || !v_cache || !pos || !out)
    return fail(GSQ_E_VALUE, "NULL pointer");
  if (!(eps >= 0.f)) return fail(GSQ_E_VALUE, "eps must be >= 0");
  AttnArgs a;
  a.qg = qg; a.k = k; a.v = v; a.q_norm_w = q_norm_w; a.k_norm_w = k_norm_w; a.inv_freq = inv_freq;
  a.kc = k_cache; a.vc = v_cache; a.pos = pos; a.out = out;
  a.qg_stride = qg_stride; a.k_stride = k_stride; a.v_stride = v_stride; a.out_stride = out_stride;
  a.B = (int)batch; a.H = (int)heads; a.Hkv = (int)kv_heads; a.hd = (int)head_dim; a.rd = (int)rotary_dim;
  a.L = (int)max_len; a.eps = eps;
  if (work) {
    a.work = work;
    a.chunk = (int)chunk;
    a.nsplit = (int)((max_len + chunk - 1) / chunk);
  }
  hipError_t e = launch_attn_decode(dtype, a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(GSQ_E_HIP, "attn_decode launch: %s", hipGetErrorString(e));
  return GSQ_OK;
}

}  // extern "C"
