// C ABI of the W4A8 engine (include/fable5_w4a8.h).
//
// Host side of the path: contexts (one HIP stream each), device-resident
// weights repacked once from the reference's row image, staging for the
// host-buffer entry points, and the reference's assertion classes mapped to
// status codes.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/fable5_w4a8.h"
#include "w4a8_internal.h"

using namespace w4a8;

struct w4a8_ctx {
  int device = 0;
  hipStream_t own = nullptr;
  hipStream_t stream = nullptr;
  int num_cu = 0;
  int grid = 0;            // persistent GEMV grid
  int grid_override = 0;
  int32_t *d_tables = nullptr;
  int32_t *d_err = nullptr;
  uint64_t *d_partials = nullptr;
  int partials_cap = 0;
  int32_t *d_result = nullptr;   // head argmax {idx, val}
  uint8_t *d_stage = nullptr;
  size_t stage_cap = 0;
  uint8_t *d_chain = nullptr;   // temporaries of device-side chains (w4a8_mlp_async)
  size_t chain_cap = 0;
  int32_t *d_topk_flags = nullptr;   // TOPK-32 look-back flags (kTopkFlagWords)
  int32_t topk_epoch = 0;            // epoch of the last TOPK-32 launch
  uint32_t spin_grid = 0, spin_lds = 0;   // polls before bounded waits give up (0: defaults)
  uint8_t *d_scratch = nullptr;   // this device's copy of `scratch` (no-alloc entry point)
  int32_t h_tables[kTableLen];
};

struct w4a8_weights {
  w4a8_ctx *ctx = nullptr;
  uint8_t *d = nullptr;
  int64_t nrows = 0;
  int64_t ntiles = 0;
  int32_t sh = 0;
  Layout L{};
  size_t bytes = 0;
};

// ---- device memory of the entry point that allocates nothing
// w4a8_head_topk32_noalloc_async keeps the head's y32 (at most 2^18 rows,
// the AMAX32 index range) and TOPK-32's chunk and super-chunk lists here
// instead of the context's chain buffer.  Every GPU the library runs on
// holds its own copy, 1.07 MiB, until the process ends; every call on one
// GPU shares it, so calls that overlap on one GPU race.  Nothing in it has
// to start at zero: the y32 is written whole before TOPK-32 reads it, and a
// list is read only after its flag carries the launch's epoch.
constexpr size_t kScratchY = sizeof(int32_t) << 18;
constexpr size_t kScratchLists = (size_t)(kTopkMaxChunks + kTopkMaxChunks / kTopkSuper) * 32 * 8;
static __device__ __align__(256) uint8_t scratch[kScratchY + kScratchLists];

static thread_local std::string g_err;

static int fail(int code, const std::string &msg) {
  g_err = msg;
  return code;
}

#define HIP_TRY(expr)                                                        \
  do {                                                                       \
    hipError_t e_ = (expr);                                                  \
    if (e_ != hipSuccess)                                                    \
      return fail(W4A8_E_HIP, std::string(#expr) + ": " + hipGetErrorString(e_)); \
  } while (0)

namespace {

struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) (void)hipSetDevice(dev);
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev)
      (void)hipSetDevice(prev);
  }
};

// The device address of this device's `scratch`, resolved once per device
// with that device current (the caller's DeviceGuard).  The array's name is
// only a host-side stand-in: host code passes this address, never the name.
int scratch_address(int device, uint8_t **out) {
  static std::mutex mu;
  static std::map<int, uint8_t *> addr;
  std::lock_guard<std::mutex> lk(mu);
  auto it = addr.find(device);
  if (it == addr.end()) {
    void *p = nullptr;
    HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(W4A8_E_HIP, "hipGetSymbolAddress(scratch) gave a null address");
    it = addr.emplace(device, (uint8_t *)p).first;
  }
  *out = it->second;
  return W4A8_OK;
}

int64_t wire_stride(int32_t K) {
  const int ng = K / kGroup;
  return (int64_t)(ng + (ng + 31) / 32) * 64;
}

// K legality and the engine envelope (w4a8_ref.py:104-105; hwmap.py:146-169)
int check_k_sh(int32_t K, int32_t sh) {
  if (K <= 0 || K % kGroup)
    return fail(W4A8_E_SHAPE, "K=" + std::to_string(K) + " must be a multiple of 128");
  if (K / kGroup > kNgMax)
    return fail(W4A8_E_ENVELOPE, "ng=" + std::to_string(K / kGroup) +
                                     " outside the engine envelope 1..96");
  if (sh < 0 || sh > 63)
    return fail(W4A8_E_ENVELOPE, "sh=" + std::to_string(sh) + " outside 0..63");
  return W4A8_OK;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

void build_tables(int32_t *t) {
  // fixedpoint.py:42-53: round(2^15 / sqrt(mid)), 256 midpoints over [1,2)
  // then 256 over [2,4).  sqrt is correctly rounded and nearbyint rounds
  // half to even like numpy.round.
  for (int i = 0; i < 256; ++i) {
    t[kRsqrtOff + i] = (int32_t)std::nearbyint(32768.0 / std::sqrt(1.0 + (i + 0.5) / 256.0));
    t[kRsqrtOff + 256 + i] =
        (int32_t)std::nearbyint(32768.0 / std::sqrt(2.0 + (i + 0.5) / 128.0));
  }
  // fixedpoint.py:128-142: sigmoid knots over [-16, 16], Q15, max 32767
  for (int i = 0; i <= 256; ++i) {
    const double x = -16.0 + 32.0 * i / 256.0;
    double v = std::nearbyint(32768.0 / (1.0 + std::exp(-x)));
    t[kSigmoidOff + i] = (int32_t)(v > 32767.0 ? 32767.0 : v);
  }
}

int ensure_stage(w4a8_ctx *c, size_t bytes) {
  if (bytes <= c->stage_cap) return W4A8_OK;
  if (c->d_stage) HIP_TRY(hipFree(c->d_stage));
  c->d_stage = nullptr;
  c->stage_cap = 0;
  size_t cap = bytes < (1u << 20) ? (1u << 20) : bytes;
  HIP_TRY(hipMalloc(&c->d_stage, cap));
  c->stage_cap = cap;
  return W4A8_OK;
}

// the context's buffer for the temporaries of device-side chains
int ensure_chain(w4a8_ctx *c, size_t bytes) {
  if (bytes <= c->chain_cap) return W4A8_OK;
  HIP_TRY(hipStreamSynchronize(c->stream));   // earlier chains may still use it
  if (c->d_chain) HIP_TRY(hipFree(c->d_chain));
  c->d_chain = nullptr;
  c->chain_cap = 0;
  HIP_TRY(hipMalloc(&c->d_chain, bytes));
  c->chain_cap = bytes;
  return W4A8_OK;
}

int ensure_partials(w4a8_ctx *c, int n) {
  if (n <= c->partials_cap) return W4A8_OK;
  if (c->d_partials) HIP_TRY(hipFree(c->d_partials));
  c->d_partials = nullptr;
  c->partials_cap = 0;
  HIP_TRY(hipMalloc(&c->d_partials, sizeof(uint64_t) * (size_t)n));
  c->partials_cap = n;
  return W4A8_OK;
}

// reads and clears the device error word (stream must be idle)
int take_err(w4a8_ctx *c) {
  int32_t h = 0;
  HIP_TRY(hipMemcpy(&h, c->d_err, sizeof(h), hipMemcpyDeviceToHost));
  if (h) {
    HIP_TRY(hipMemset(c->d_err, 0, sizeof(int32_t)));
    // a wait that gave up leaves the launch's results undefined (an
    // overflow found after it is one of them), so it is reported first
    if (h & 2)
      return fail(W4A8_E_HIP, "a persistent plan's wait for other workgroups timed out "
                            "(are all of its workgroups resident? another long-running "
                            "kernel on the GPU can hold CUs; W4A8_PLAN_PERSISTENT_COOP "
                            "guarantees residency)");
    if (h & 4)
      return fail(W4A8_E_HIP, "a wait between wavefronts of one workgroup timed out");
    if (h & 8)
      return fail(W4A8_E_HIP, "TOPK-32's wait for the lists of earlier chunks timed out");
    if (h & 1) return fail(W4A8_E_Y32_OVF, "y32 overflow — sh miscomputed");
    if (h & 16) return fail(W4A8_E_RANGE, "MOVX source is not int8-packed");
  }
  return W4A8_OK;
}

int grid_for(w4a8_ctx *c, int64_t tiles) {
  const int g = c->grid_override > 0 ? c->grid_override : c->grid;
  return (int)(tiles < g ? tiles : g);
}

// fills prologue fields and validates them
int set_prologue(w4a8_ctx *c, GemvParams &P, int32_t K, int32_t prologue,
                 const void *x, const int16_t *norm_w, int32_t in_f,
                 int32_t one_plus, int32_t e_x) {
  if (prologue < PRO_X8 || prologue > PRO_RMSNORM_DYNQ8)
    return fail(W4A8_E_ARG, "unknown prologue " + std::to_string(prologue));
  if (!x || !aligned16(x)) return fail(W4A8_E_ARG, "x must be a 16-byte aligned pointer");
  if (prologue == PRO_RMSNORM_DYNQ8) {
    if (!norm_w || !aligned16(norm_w))
      return fail(W4A8_E_ARG, "norm_w must be a 16-byte aligned pointer");
    if ((K & (K - 1)) != 0)
      return fail(W4A8_E_RANGE, "rmsnorm_fx: n=" + std::to_string(K) +
                                    " is not a power of 2");
    if (K > 8192)
      return fail(W4A8_E_RANGE, "rmsnorm_fx: n=" + std::to_string(K) + " > 8192");
    if (in_f < 0 || in_f > kRmsInFMax)
      return fail(W4A8_E_RANGE, "rmsnorm_fx: in_f=" + std::to_string(in_f) +
                                    " outside 0.." + std::to_string(kRmsInFMax));
  }
  P.K = K;
  P.NG = K / kGroup;
  P.nblk = (P.NG + kGroupsPerBlock - 1) / kGroupsPerBlock;
  P.tile_bytes = layout_for(K).tile_bytes;
  P.pro = prologue;
  P.x = x;
  P.norm_w = norm_w;
  P.in_f = in_f;
  P.one_plus = one_plus ? 1 : 0;
  P.e_x_given = e_x;
  P.tables = c->d_tables;
  P.err = c->d_err;
  return W4A8_OK;
}

int check_epilogue(int32_t epi) {
  if (epi < EPI_Y32 || epi > EPI_SHIFT_I64)
    return fail(W4A8_E_ARG, "unknown epilogue " + std::to_string(epi));
  return W4A8_OK;
}

size_t out_elem(int32_t epi) {
  switch (epi) {
    case EPI_MOVY_I16:
    case EPI_SILU32: return 2;
    case EPI_SHIFT_I64: return 8;
    default: return 4;
  }
}

int site_params(w4a8_ctx *c, GemvParams &P, int32_t nmat,
                const w4a8_weights *const *w, const int32_t *epi, const int32_t *p0,
                void *const *out, int32_t prologue, const void *x,
                const int16_t *norm_w, int32_t in_f, int32_t one_plus, int32_t e_x,
                int8_t *x8_out, int32_t *e_x_out, int16_t *xn_out) {
  if (nmat < 1 || nmat > kMaxJobs)
    return fail(W4A8_E_ARG, "site holds 1.." + std::to_string(kMaxJobs) + " matrices");
  P = GemvParams{};
  if (!w[0]) return fail(W4A8_E_ARG, "null weights");
  const int32_t K = w[0]->L.K;
  int rc = set_prologue(c, P, K, prologue, x, norm_w, in_f, one_plus, e_x);
  if (rc) return rc;
  int64_t tiles = 0;
  for (int i = 0; i < nmat; ++i) {
    if (!w[i] || !out[i]) return fail(W4A8_E_ARG, "null weights/output");
    if (w[i]->L.K != K) return fail(W4A8_E_SHAPE, "matrices of one site must share K");
    if ((rc = check_epilogue(epi[i]))) return rc;
    P.job[i].w = w[i]->d;
    P.job[i].out = out[i];
    P.job[i].nrows = (int32_t)w[i]->nrows;
    P.job[i].tile0 = P.tile0[i] = (int32_t)tiles;
    P.job[i].sh = w[i]->sh;
    P.job[i].epi = epi[i];
    P.job[i].p0 = p0[i];
    tiles += w[i]->ntiles;
  }
  P.njobs = nmat;
  P.total_tiles = (int32_t)tiles;
  P.x8_out = x8_out;
  P.e_x_out = e_x_out;
  P.xn_out = xn_out;
  P.partials = nullptr;
  return W4A8_OK;
}

int site_launch(w4a8_ctx *c, int32_t nmat, const w4a8_weights *const *w,
                const int32_t *epi, const int32_t *p0, void *const *out,
                int32_t prologue, const void *x, const int16_t *norm_w,
                int32_t in_f, int32_t one_plus, int32_t e_x, int8_t *x8_out,
                int32_t *e_x_out, int16_t *xn_out) {
  GemvParams P;
  int rc = site_params(c, P, nmat, w, epi, p0, out, prologue, x, norm_w, in_f,
                       one_plus, e_x, x8_out, e_x_out, xn_out);
  if (rc) return rc;
  DeviceGuard g(c->device);
  HIP_TRY(launch_gemv(P, grid_for(c, P.total_tiles), c->stream));
  return W4A8_OK;
}

int head_params(w4a8_ctx *c, GemvParams &P, const w4a8_weights *w, int32_t prologue,
                const void *x, const int16_t *norm_w, int32_t in_f,
                int32_t one_plus, int32_t e_x) {
  if (!w) return fail(W4A8_E_ARG, "null weights");
  if (w->nrows > (1 << 18))
    return fail(W4A8_E_RANGE, "vocab " + std::to_string(w->nrows) +
                                  " exceeds the 18-bit AMAX32 index (2^18)");
  P = GemvParams{};
  int rc = set_prologue(c, P, w->L.K, prologue, x, norm_w, in_f, one_plus, e_x);
  if (rc) return rc;
  P.job[0].w = w->d;
  P.job[0].out = nullptr;
  P.job[0].nrows = (int32_t)w->nrows;
  P.job[0].tile0 = P.tile0[0] = 0;
  P.job[0].sh = w->sh;
  P.job[0].epi = EPI_ARGMAX;
  P.job[0].p0 = 0;
  P.njobs = 1;
  P.total_tiles = (int32_t)w->ntiles;
  return W4A8_OK;
}

int head_launch(w4a8_ctx *c, const w4a8_weights *w, int32_t prologue,
                const void *x, const int16_t *norm_w, int32_t in_f,
                int32_t one_plus, int32_t e_x, int32_t *d_result) {
  GemvParams P;
  int rc = head_params(c, P, w, prologue, x, norm_w, in_f, one_plus, e_x);
  if (rc) return rc;
  const int grid = grid_for(c, w->ntiles);
  if ((rc = ensure_partials(c, grid))) return rc;
  P.partials = c->d_partials;
  DeviceGuard g(c->device);
  HIP_TRY(launch_gemv(P, grid, c->stream));
  HIP_TRY(launch_argmax_final(c->d_partials, grid, d_result, c->stream));
  return W4A8_OK;
}

}  // namespace

extern "C" {

const char *w4a8_version(void) { return "fable5-w4a8 0.1 gfx950"; }

const char *w4a8_last_error(void) { return g_err.c_str(); }

int w4a8_ctx_create(int32_t device, w4a8_ctx **out) {
  if (!out) return fail(W4A8_E_ARG, "null out");
  *out = nullptr;
  int ndev = 0;
  HIP_TRY(hipGetDeviceCount(&ndev));
  if (device < 0 || device >= ndev)
    return fail(W4A8_E_ARG, "no HIP device " + std::to_string(device));
  DeviceGuard g(device);
  w4a8_ctx *c = new w4a8_ctx();
  c->device = device;
  int rc = W4A8_OK;
  do {
    hipError_t e;
    if ((e = hipStreamCreateWithFlags(&c->own, hipStreamNonBlocking)) != hipSuccess) {
      rc = fail(W4A8_E_HIP, std::string("hipStreamCreate: ") + hipGetErrorString(e));
      break;
    }
    c->stream = c->own;
    if ((e = hipDeviceGetAttribute(&c->num_cu, hipDeviceAttributeMultiprocessorCount,
                                   device)) != hipSuccess) {
      rc = fail(W4A8_E_HIP, hipGetErrorString(e));
      break;
    }
    c->grid = c->num_cu * gemv_max_blocks_per_cu();
    build_tables(c->h_tables);
    if ((e = hipMalloc(&c->d_tables, sizeof(int32_t) * kTableLen)) != hipSuccess ||
        (e = hipMemcpy(c->d_tables, c->h_tables, sizeof(int32_t) * kTableLen,
                       hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipMalloc(&c->d_err, 64)) != hipSuccess ||
        (e = hipMemset(c->d_err, 0, 64)) != hipSuccess ||
        (e = hipMalloc(&c->d_result, 64)) != hipSuccess ||
        (e = hipMalloc(&c->d_topk_flags, sizeof(int32_t) * kTopkFlagWords)) != hipSuccess ||
        (e = hipMemset(c->d_topk_flags, 0, sizeof(int32_t) * kTopkFlagWords)) != hipSuccess) {
      rc = fail(W4A8_E_HIP, hipGetErrorString(e));
      break;
    }
    rc = scratch_address(device, &c->d_scratch);
  } while (0);
  if (rc) {
    w4a8_ctx_destroy(c);
    return rc;
  }
  *out = c;
  return W4A8_OK;
}

int w4a8_ctx_destroy(w4a8_ctx *c) {
  if (!c) return W4A8_OK;
  DeviceGuard g(c->device);
  if (c->own) (void)hipStreamSynchronize(c->own);
  if (c->stream && c->stream != c->own) (void)hipStreamSynchronize(c->stream);
  (void)hipFree(c->d_tables);
  (void)hipFree(c->d_err);
  (void)hipFree(c->d_partials);
  (void)hipFree(c->d_result);
  (void)hipFree(c->d_stage);
  (void)hipFree(c->d_chain);
  (void)hipFree(c->d_topk_flags);
  if (c->own) (void)hipStreamDestroy(c->own);
  delete c;
  return W4A8_OK;
}

int w4a8_ctx_set_stream(w4a8_ctx *c, void *s) {
  if (!c) return fail(W4A8_E_ARG, "null ctx");
  c->stream = s ? (hipStream_t)s : c->own;
  return W4A8_OK;
}

int w4a8_ctx_sync(w4a8_ctx *c) {
  if (!c) return fail(W4A8_E_ARG, "null ctx");
  DeviceGuard g(c->device);
  HIP_TRY(hipStreamSynchronize(c->stream));
  return take_err(c);
}

int w4a8_ctx_info(const w4a8_ctx *c, int32_t *num_cu, int32_t *grid) {
  if (!c) return fail(W4A8_E_ARG, "null ctx");
  if (num_cu) *num_cu = c->num_cu;
  if (grid) *grid = c->grid_override > 0 ? c->grid_override : c->grid;
  return W4A8_OK;
}

int w4a8_read_ceiling(w4a8_ctx *c, const void *d_buf, int64_t nbytes, int32_t grid, int32_t n,
                      float *ms) {
  if (!c || !d_buf || !ms || n < 1 || nbytes < 16 || nbytes % 16 || grid < 0)
    return fail(W4A8_E_ARG, "w4a8_read_ceiling: bad argument");
  DeviceGuard g(c->device);
  if (grid == 0) grid = 8 * c->num_cu;
  uint32_t *sink = nullptr;
  HIP_TRY(hipMalloc(&sink, sizeof(uint32_t) * (size_t)grid));
  std::vector<hipEvent_t> ev(2 * (size_t)n, nullptr);
  int rc = W4A8_OK;
  for (auto &e : ev)
    if (!rc && hipEventCreate(&e) != hipSuccess) rc = fail(W4A8_E_HIP, "hipEventCreate");
  for (int i = 0; !rc && i < n; ++i)
    if (launch_read(d_buf, nbytes, sink, grid, c->stream, ev[2 * i], ev[2 * i + 1]) !=
        hipSuccess)
      rc = fail(W4A8_E_HIP, "read_kernel launch");
  if (!rc && hipStreamSynchronize(c->stream) != hipSuccess) rc = fail(W4A8_E_HIP, "sync");
  for (int i = 0; !rc && i < n; ++i)
    if (hipEventElapsedTime(&ms[i], ev[2 * i], ev[2 * i + 1]) != hipSuccess)
      rc = fail(W4A8_E_HIP, "hipEventElapsedTime");
  for (auto &e : ev)
    if (e) (void)hipEventDestroy(e);
  (void)hipFree(sink);
  return rc;
}

int w4a8_ctx_set_spin_limit(w4a8_ctx *c, uint32_t grid_polls, uint32_t lds_polls) {
  if (!c) return fail(W4A8_E_ARG, "null ctx");
  c->spin_grid = grid_polls;
  c->spin_lds = lds_polls;
  return W4A8_OK;
}

int w4a8_ctx_set_grid(w4a8_ctx *c, int32_t grid) {
  if (!c || grid < 0) return fail(W4A8_E_ARG, "bad ctx/grid");
  c->grid_override = grid;
  return W4A8_OK;
}

int w4a8_tables(w4a8_ctx *c, int32_t *rsqrt512, int32_t *sigmoid257) {
  if (!c) return fail(W4A8_E_ARG, "null ctx");
  // read back what the device actually holds
  int32_t t[kTableLen];
  DeviceGuard g(c->device);
  HIP_TRY(hipMemcpy(t, c->d_tables, sizeof(t), hipMemcpyDeviceToHost));
  if (rsqrt512) memcpy(rsqrt512, t + kRsqrtOff, 512 * sizeof(int32_t));
  if (sigmoid257) memcpy(sigmoid257, t + kSigmoidOff, 257 * sizeof(int32_t));
  return W4A8_OK;
}

// ------------------------------------------------------------------ weights
static int upload_common(w4a8_ctx *c, const uint8_t *img, bool host, int64_t nrows,
                         int32_t K, int32_t sh, w4a8_weights **out) {
  if (!c || !img || !out) return fail(W4A8_E_ARG, "null argument");
  *out = nullptr;
  int rc = check_k_sh(K, sh);
  if (rc) return rc;
  if (nrows < 1 || nrows > (int64_t)1 << 30)
    return fail(W4A8_E_SHAPE, "nrows=" + std::to_string(nrows) + " out of range");
  DeviceGuard g(c->device);
  w4a8_weights *w = new w4a8_weights();
  w->ctx = c;
  w->nrows = nrows;
  w->ntiles = (nrows + kTileRows - 1) / kTileRows;
  w->sh = sh;
  w->L = layout_for(K);
  w->bytes = (size_t)(w->ntiles * w->L.tile_bytes);
  const int64_t stride = wire_stride(K);
  hipError_t e = hipMalloc(&w->d, w->bytes);
  if (e != hipSuccess) {
    delete w;
    return fail(W4A8_E_HIP, std::string("hipMalloc weights: ") + hipGetErrorString(e));
  }
  const uint8_t *src = img;
  uint8_t *tmp = nullptr;
  if (host || !aligned16(img)) {
    e = hipMalloc(&tmp, (size_t)(nrows * stride));
    if (e == hipSuccess)
      e = hipMemcpyAsync(tmp, img, (size_t)(nrows * stride),
                         host ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice,
                         c->stream);
    src = tmp;
  }
  if (e == hipSuccess) e = launch_repack(src, nrows, w->L, stride, w->d, c->stream);
  if (e == hipSuccess && (host || tmp)) e = hipStreamSynchronize(c->stream);
  if (tmp) (void)hipFree(tmp);
  if (e != hipSuccess) {
    (void)hipFree(w->d);
    delete w;
    return fail(W4A8_E_HIP, std::string("weights upload: ") + hipGetErrorString(e));
  }
  *out = w;
  return W4A8_OK;
}

int w4a8_weights_upload(w4a8_ctx *c, const uint8_t *img, int64_t nrows, int32_t K,
                        int32_t sh, w4a8_weights **out) {
  return upload_common(c, img, true, nrows, K, sh, out);
}

int w4a8_weights_upload_async(w4a8_ctx *c, const uint8_t *d_img, int64_t nrows,
                              int32_t K, int32_t sh, w4a8_weights **out) {
  return upload_common(c, d_img, false, nrows, K, sh, out);
}

int w4a8_weights_download(w4a8_ctx *c, const w4a8_weights *w, uint8_t *img) {
  if (!c || !w || !img) return fail(W4A8_E_ARG, "null argument");
  DeviceGuard g(c->device);
  const int64_t stride = wire_stride(w->L.K);
  const size_t n = (size_t)(w->nrows * stride);
  int rc = ensure_stage(c, n);
  if (rc) return rc;
  HIP_TRY(launch_unpack(w->d, w->nrows, w->L, stride, c->d_stage, c->stream));
  HIP_TRY(hipMemcpyAsync(img, c->d_stage, n, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return W4A8_OK;
}

int w4a8_weights_info(const w4a8_weights *w, int64_t *nrows, int32_t *K, int32_t *sh,
                      int64_t *bytes) {
  if (!w) return fail(W4A8_E_ARG, "null weights");
  if (nrows) *nrows = w->nrows;
  if (K) *K = w->L.K;
  if (sh) *sh = w->sh;
  if (bytes) *bytes = (int64_t)w->bytes;
  return W4A8_OK;
}

int w4a8_weights_free(w4a8_weights *w) {
  if (!w) return W4A8_OK;
  DeviceGuard g(w->ctx->device);
  (void)hipStreamSynchronize(w->ctx->stream);
  (void)hipFree(w->d);
  delete w;
  return W4A8_OK;
}

// --------------------------------------------------------- elementwise ops
int w4a8_rshift_round(w4a8_ctx *c, const int64_t *v, int64_t n, int32_t s, int64_t *out) {
  if (!c || (n > 0 && (!v || !out)) || n < 0) return fail(W4A8_E_ARG, "bad argument");
  if (s < -63 || s > 63) return fail(W4A8_E_RANGE, "shift outside -63..63");
  if (n == 0) return W4A8_OK;
  DeviceGuard g(c->device);
  int rc = ensure_stage(c, (size_t)n * 16);
  if (rc) return rc;
  int64_t *d_in = (int64_t *)c->d_stage, *d_out = d_in + n;
  HIP_TRY(hipMemcpyAsync(d_in, v, n * 8, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(launch_rshift_round(d_in, n, s, d_out, c->stream));
  HIP_TRY(hipMemcpyAsync(out, d_out, n * 8, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return W4A8_OK;
}

static int vec_prologue(w4a8_ctx *c, int32_t pro, const int16_t *x16,
                        const int16_t *w_q14, int32_t n, int32_t in_f,
                        int32_t one_plus, int8_t *x8, int32_t *e, int16_t *xn) {
  if (!c || !x16) return fail(W4A8_E_ARG, "null argument");
  if (n < 1 || n > kKMax || n % 8)
    return fail(W4A8_E_RANGE, "vector length " + std::to_string(n) +
                                  " must be a multiple of 8 in 8..12288");
  DeviceGuard g(c->device);
  const size_t nb = (size_t)n * 2;
  int rc = ensure_stage(c, 4 * nb + 64);
  if (rc) return rc;
  uint8_t *base = c->d_stage;
  int16_t *d_x = (int16_t *)base;
  int16_t *d_w = (int16_t *)(base + nb);
  int16_t *d_xn = (int16_t *)(base + 2 * nb);
  int8_t *d_x8 = (int8_t *)(base + 3 * nb);
  int32_t *d_e = (int32_t *)(base + 4 * nb);
  HIP_TRY(hipMemcpyAsync(d_x, x16, nb, hipMemcpyHostToDevice, c->stream));
  if (pro == PRO_RMSNORM_DYNQ8)
    HIP_TRY(hipMemcpyAsync(d_w, w_q14, nb, hipMemcpyHostToDevice, c->stream));
  GemvParams P{};
  if (pro == PRO_RMSNORM_DYNQ8) {
    if ((n & (n - 1)) != 0)
      return fail(W4A8_E_RANGE, "rmsnorm_fx: n=" + std::to_string(n) + " is not a power of 2");
    if (n > 8192) return fail(W4A8_E_RANGE, "rmsnorm_fx: n > 8192");
    if (in_f < 0 || in_f > kRmsInFMax)
      return fail(W4A8_E_RANGE, "rmsnorm_fx: in_f=" + std::to_string(in_f) +
                                    " outside 0.." + std::to_string(kRmsInFMax));
  }
  P.K = n;
  P.NG = 0;
  P.pro = pro;
  P.x = d_x;
  P.norm_w = d_w;
  P.in_f = in_f;
  P.one_plus = one_plus ? 1 : 0;
  P.tables = c->d_tables;
  P.err = c->d_err;
  P.x8_out = d_x8;
  P.e_x_out = d_e;
  P.xn_out = d_xn;
  HIP_TRY(launch_vec_prologue(P, c->stream));
  if (x8) HIP_TRY(hipMemcpyAsync(x8, d_x8, n, hipMemcpyDeviceToHost, c->stream));
  if (e) HIP_TRY(hipMemcpyAsync(e, d_e, 4, hipMemcpyDeviceToHost, c->stream));
  if (xn) HIP_TRY(hipMemcpyAsync(xn, d_xn, nb, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return W4A8_OK;
}

int w4a8_dynq8(w4a8_ctx *c, const int16_t *x16, int32_t n, int8_t *x8, int32_t *e) {
  return vec_prologue(c, PRO_DYNQ8, x16, nullptr, n, 0, 0, x8, e, nullptr);
}

int w4a8_rmsnorm(w4a8_ctx *c, const int16_t *x16, const int16_t *w_q14, int32_t n,
                 int32_t in_f, int32_t one_plus, int16_t *out) {
  if (!w_q14 || !out) return fail(W4A8_E_ARG, "null argument");
  return vec_prologue(c, PRO_RMSNORM_DYNQ8, x16, w_q14, n, in_f, one_plus, nullptr,
                      nullptr, out);
}

int w4a8_movy(w4a8_ctx *c, const int32_t *y32, int64_t n, int32_t shift, int32_t mode,
              void *out) {
  if (!c || n < 0 || (n > 0 && (!y32 || !out))) return fail(W4A8_E_ARG, "bad argument");
  if (mode != W4A8_MOVY_INT16 && mode != W4A8_MOVY_PAIRS32)
    return fail(W4A8_E_ARG, "unknown MOVY mode");
  if (n == 0) return W4A8_OK;
  DeviceGuard g(c->device);
  const size_t ob = mode == W4A8_MOVY_INT16 ? 2 : 4;
  int rc = ensure_stage(c, (size_t)n * (4 + ob) + 16);
  if (rc) return rc;
  int32_t *d_y = (int32_t *)c->d_stage;
  void *d_o = c->d_stage + (((size_t)n * 4 + 15) & ~(size_t)15);
  HIP_TRY(hipMemcpyAsync(d_y, y32, n * 4, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(launch_movy(d_y, n, shift, mode, d_o, c->stream));
  HIP_TRY(hipMemcpyAsync(out, d_o, n * ob, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return W4A8_OK;
}

int w4a8_movy_async(w4a8_ctx *c, const int32_t *d_y32, int64_t n, int32_t shift,
                    int32_t mode, void *d_out) {
  if (!c || n < 0 || (n > 0 && (!d_y32 || !d_out))) return fail(W4A8_E_ARG, "bad argument");
  if (mode != W4A8_MOVY_INT16 && mode != W4A8_MOVY_PAIRS32)
    return fail(W4A8_E_ARG, "unknown MOVY mode");
  if (((uintptr_t)d_y32 & 3) || ((uintptr_t)d_out & (mode == W4A8_MOVY_INT16 ? 1 : 3)))
    return fail(W4A8_E_ARG, "MOVY: y32 and pairs32 output must be 4-byte aligned, int16 "
                            "output 2-byte aligned");
  if (n == 0) return W4A8_OK;
  DeviceGuard g(c->device);
  HIP_TRY(launch_movy(d_y32, n, shift, mode, d_out, c->stream));
  return W4A8_OK;
}

int w4a8_movx_async(w4a8_ctx *c, const int16_t *d_src, int64_t n, int8_t *d_x8) {
  if (!c || n < 0 || (n > 0 && (!d_src || !d_x8))) return fail(W4A8_E_ARG, "bad argument");
  if (((uintptr_t)d_src & 1) || ((uintptr_t)d_x8 & 3))
    return fail(W4A8_E_ARG, "MOVX: source must be 2-byte and x window 4-byte aligned");
  if (n == 0) return W4A8_OK;
  DeviceGuard g(c->device);
  HIP_TRY(launch_movx(d_src, n, d_x8, c->d_err, c->stream));
  return W4A8_OK;
}

int w4a8_alu(w4a8_ctx *c, int32_t op, const int32_t *y32, const int16_t *b, int64_t n,
             int32_t p0, void *out) {
  if (!c || n < 0 || (n > 0 && (!y32 || !out))) return fail(W4A8_E_ARG, "bad argument");
  if (op != W4A8_ALU_SHIFT32 && op != W4A8_ALU_SILU32 && op != W4A8_ALU_EMUL32 &&
      op != W4A8_ALU_SHIFT32W)
    return fail(W4A8_E_ARG, "unsupported ALU op " + std::to_string(op));
  if (op == W4A8_ALU_EMUL32 && !b) return fail(W4A8_E_ARG, "EMUL32 needs b");
  if (n > 16383)
    return fail(W4A8_E_RANGE, "ALU count " + std::to_string(n) +
                                  " does not fit ARG0[17:4] (max 16383)");
  if (n == 0) return W4A8_OK;
  DeviceGuard g(c->device);
  const size_t ob = op == W4A8_ALU_SHIFT32W ? 4 : 2;
  const size_t a4 = ((size_t)n * 4 + 15) & ~(size_t)15, a2 = ((size_t)n * 2 + 15) & ~(size_t)15;
  int rc = ensure_stage(c, a4 + a2 + n * ob + 16);
  if (rc) return rc;
  int32_t *d_y = (int32_t *)c->d_stage;
  int16_t *d_b = (int16_t *)(c->d_stage + a4);
  void *d_o = c->d_stage + a4 + a2;
  HIP_TRY(hipMemcpyAsync(d_y, y32, n * 4, hipMemcpyHostToDevice, c->stream));
  if (b) HIP_TRY(hipMemcpyAsync(d_b, b, n * 2, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(launch_alu(op, d_y, d_b, n, p0, c->d_tables, d_o, c->stream));
  HIP_TRY(hipMemcpyAsync(out, d_o, n * ob, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return W4A8_OK;
}

// ------------------------------------------------------------- matvec (host)
int w4a8_matvec_fused(w4a8_ctx *c, const w4a8_weights *w, int32_t prologue,
                      const void *x, const int16_t *norm_w, int32_t in_f,
                      int32_t one_plus, int32_t epilogue, int32_t p0, void *out,
                      int8_t *x8_out, int32_t *e_x_io, int16_t *xn_out) {
  if (!c || !w || !x || !out) return fail(W4A8_E_ARG, "null argument");
  int rc = check_epilogue(epilogue);
  if (rc) return rc;
  if (prologue == PRO_X8 && !e_x_io && epilogue != EPI_Y32)
    return fail(W4A8_E_ARG, "PRO_X8 with a shifting epilogue needs e_x");
  DeviceGuard g(c->device);
  const int32_t K = w->L.K;
  const size_t xb = prologue == PRO_X8 ? (size_t)K : (size_t)K * 2;
  const size_t A = 256;
  auto up = [&](size_t v) { return (v + A - 1) & ~(A - 1); };
  const size_t ob = out_elem(epilogue) * (size_t)w->nrows;
  const size_t o_x = 0, o_w = up(xb), o_out = o_w + up((size_t)K * 2),
               o_x8 = o_out + up(ob), o_e = o_x8 + up(K), o_xn = o_e + A,
               total = o_xn + up((size_t)K * 2);
  if ((rc = ensure_stage(c, total))) return rc;
  uint8_t *s = c->d_stage;
  HIP_TRY(hipMemcpyAsync(s + o_x, x, xb, hipMemcpyHostToDevice, c->stream));
  if (prologue == PRO_RMSNORM_DYNQ8) {
    if (!norm_w) return fail(W4A8_E_ARG, "PRO_RMSNORM_DYNQ8 needs norm_w");
    HIP_TRY(hipMemcpyAsync(s + o_w, norm_w, (size_t)K * 2, hipMemcpyHostToDevice,
                           c->stream));
  }
  const int32_t ex_in = (prologue == PRO_X8 && e_x_io) ? *e_x_io : 0;
  const int32_t ep = epilogue;
  void *d_out = s + o_out;
  rc = site_launch(c, 1, &w, &ep, &p0, &d_out, prologue, s + o_x,
                   (const int16_t *)(s + o_w), in_f, one_plus, ex_in,
                   (int8_t *)(s + o_x8), (int32_t *)(s + o_e), (int16_t *)(s + o_xn));
  if (rc) return rc;
  HIP_TRY(hipMemcpyAsync(out, d_out, ob, hipMemcpyDeviceToHost, c->stream));
  if (x8_out) HIP_TRY(hipMemcpyAsync(x8_out, s + o_x8, K, hipMemcpyDeviceToHost, c->stream));
  if (e_x_io) HIP_TRY(hipMemcpyAsync(e_x_io, s + o_e, 4, hipMemcpyDeviceToHost, c->stream));
  if (xn_out && prologue == PRO_RMSNORM_DYNQ8)
    HIP_TRY(hipMemcpyAsync(xn_out, s + o_xn, (size_t)K * 2, hipMemcpyDeviceToHost,
                           c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return take_err(c);
}

int w4a8_matvec_y32(w4a8_ctx *c, const w4a8_weights *w, const int8_t *x8, int32_t *y32) {
  int32_t ex = 0;
  return w4a8_matvec_fused(c, w, PRO_X8, x8, nullptr, 0, 0, EPI_Y32, 0, y32, nullptr,
                           &ex, nullptr);
}

int w4a8_head_argmax(w4a8_ctx *c, const w4a8_weights *w, int32_t prologue, const void *x,
                     const int16_t *norm_w, int32_t in_f, int32_t one_plus,
                     int32_t *idx, int32_t *val) {
  if (!c || !w || !x) return fail(W4A8_E_ARG, "null argument");
  DeviceGuard g(c->device);
  const int32_t K = w->L.K;
  const size_t xb = prologue == PRO_X8 ? (size_t)K : (size_t)K * 2;
  const size_t o_w = (xb + 255) & ~(size_t)255;
  int rc = ensure_stage(c, o_w + (size_t)K * 2 + 256);
  if (rc) return rc;
  uint8_t *s = c->d_stage;
  HIP_TRY(hipMemcpyAsync(s, x, xb, hipMemcpyHostToDevice, c->stream));
  if (prologue == PRO_RMSNORM_DYNQ8 && norm_w)
    HIP_TRY(hipMemcpyAsync(s + o_w, norm_w, (size_t)K * 2, hipMemcpyHostToDevice,
                           c->stream));
  rc = head_launch(c, w, prologue, s, (const int16_t *)(s + o_w), in_f, one_plus, 0,
                   c->d_result);
  if (rc) return rc;
  int32_t h[2];
  HIP_TRY(hipMemcpyAsync(h, c->d_result, 8, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  if ((rc = take_err(c))) return rc;
  if (idx) *idx = h[0];
  if (val) *val = h[1];
  return W4A8_OK;
}

int w4a8_matmul_y32(w4a8_ctx *c, const w4a8_weights *w, const int8_t *x8, int32_t B,
                    int32_t *y32) {
  if (!c || !w || !x8 || !y32) return fail(W4A8_E_ARG, "null argument");
  if (B < 1 || B > 64) return fail(W4A8_E_RANGE, "batch must be 1..64");
  DeviceGuard g(c->device);
  const int32_t K = w->L.K;
  const size_t xb = (size_t)B * K, yb = (size_t)B * w->nrows * 4;
  const size_t o_y = (xb + 255) & ~(size_t)255;
  int rc = ensure_stage(c, o_y + yb);
  if (rc) return rc;
  HIP_TRY(hipMemcpyAsync(c->d_stage, x8, xb, hipMemcpyHostToDevice, c->stream));
  rc = w4a8_matmul_y32_async(c, w, (const int8_t *)c->d_stage, B,
                             (int32_t *)(c->d_stage + o_y));
  if (rc) return rc;
  HIP_TRY(hipMemcpyAsync(y32, c->d_stage + o_y, yb, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return take_err(c);
}

// ----------------------------------------------------------- async variants
int w4a8_matvec_fused_async(w4a8_ctx *c, const w4a8_weights *w, int32_t prologue,
                            const void *d_x, const int16_t *d_norm_w, int32_t in_f,
                            int32_t one_plus, int32_t e_x, int32_t epilogue, int32_t p0,
                            void *d_out, int8_t *d_x8_out, int32_t *d_e_x_out,
                            int16_t *d_xn_out) {
  if (!c || !w) return fail(W4A8_E_ARG, "null argument");
  return site_launch(c, 1, &w, &epilogue, &p0, &d_out, prologue, d_x, d_norm_w, in_f,
                     one_plus, e_x, d_x8_out, d_e_x_out, d_xn_out);
}

int w4a8_site_async(w4a8_ctx *c, int32_t nmat, const w4a8_weights *const *w,
                    const int32_t *epilogue, const int32_t *p0, void *const *d_out,
                    int32_t prologue, const void *d_x, const int16_t *d_norm_w,
                    int32_t in_f, int32_t one_plus, int32_t e_x, int8_t *d_x8_out,
                    int32_t *d_e_x_out, int16_t *d_xn_out) {
  if (!c || !w || !epilogue || !p0 || !d_out) return fail(W4A8_E_ARG, "null argument");
  return site_launch(c, nmat, w, epilogue, p0, d_out, prologue, d_x, d_norm_w, in_f,
                     one_plus, e_x, d_x8_out, d_e_x_out, d_xn_out);
}

int w4a8_head_argmax_async(w4a8_ctx *c, const w4a8_weights *w, int32_t prologue,
                           const void *d_x, const int16_t *d_norm_w, int32_t in_f,
                           int32_t one_plus, int32_t e_x, int32_t *d_result) {
  if (!c || !w || !d_result) return fail(W4A8_E_ARG, "null argument");
  return head_launch(c, w, prologue, d_x, d_norm_w, in_f, one_plus, e_x, d_result);
}

int w4a8_matmul_y32_async(w4a8_ctx *c, const w4a8_weights *w, const int8_t *d_x8,
                          int32_t B, int32_t *d_y32) {
  if (!c || !w || !d_x8 || !d_y32) return fail(W4A8_E_ARG, "null argument");
  if (B < 1 || B > 64) return fail(W4A8_E_RANGE, "batch must be 1..64");
  if (!aligned16(d_x8)) return fail(W4A8_E_ARG, "x8 must be 16-byte aligned");
  DeviceGuard g(c->device);
  HIP_TRY(launch_matmul(w->d, (int32_t)w->nrows, w->L, w->sh, d_x8, B, d_y32, c->d_err,
                        c->stream));
  return W4A8_OK;
}

int w4a8_matmul_y32_multi_async(w4a8_ctx *c, int32_t n, const w4a8_weights *const *w,
                                const int8_t *const *d_x8, int32_t B, int32_t *const *d_y32) {
  if (!c || !w || !d_x8 || !d_y32) return fail(W4A8_E_ARG, "null argument");
  if (n < 1 || n > kMmJobs)
    return fail(W4A8_E_RANGE, "matmul_multi: 1.." + std::to_string(kMmJobs) + " matrices");
  if (B < 1 || B > 64) return fail(W4A8_E_RANGE, "batch must be 1..64");
  MmJobSpec jobs[kMmJobs];
  for (int i = 0; i < n; ++i) {
    if (!w[i] || !d_x8[i] || !d_y32[i]) return fail(W4A8_E_ARG, "null weights / x8 / y32");
    if (!aligned16(d_x8[i])) return fail(W4A8_E_ARG, "x8 must be 16-byte aligned");
    jobs[i] = MmJobSpec{w[i]->d, (int32_t)w[i]->nrows, w[i]->L, w[i]->sh, d_x8[i], d_y32[i]};
  }
  DeviceGuard g(c->device);
  HIP_TRY(launch_matmul_multi(jobs, n, B, c->d_err, c->stream));
  return W4A8_OK;
}

// ------------------------------------------------------------ matmul plan
// Up to kMmPlanJobs matrices for the same B tokens, their records in a
// device table written at the first run after the last add: one launch of
// matmul_kernel per run, the weight stream running on across every matrix.
struct w4a8_mplan {
  w4a8_ctx *ctx = nullptr;
  int32_t B = 0;
  std::vector<MmJobSpec> jobs;
  void *d_table = nullptr;
  MmPlanCfg cfg{};
  bool built = false;
  uint8_t *d_part = nullptr;  // the K-split jobs' slice sums
  void *d_fin = nullptr;      // their finishing records
  int nfin = 0;
  int64_t fin_max = 0;        // the largest B * nrows among them
  // buffers of earlier builds: a graph the caller captured from an earlier
  // run still points at them, so they are freed only by destroy
  std::vector<void *> retired;
};

int w4a8_mplan_create(w4a8_ctx *c, int32_t B, w4a8_mplan **out) {
  if (!c || !out) return fail(W4A8_E_ARG, "null argument");
  if (B < 1 || B > 64) return fail(W4A8_E_RANGE, "batch must be 1..64");
  w4a8_mplan *p = new w4a8_mplan();
  p->ctx = c;
  p->B = B;
  *out = p;
  return W4A8_OK;
}

int w4a8_mplan_add(w4a8_mplan *p, const w4a8_weights *w, const int8_t *d_x8, int32_t *d_y32) {
  if (!p || !w || !d_x8 || !d_y32) return fail(W4A8_E_ARG, "null weights / x8 / y32");
  if (!aligned16(d_x8)) return fail(W4A8_E_ARG, "x8 must be 16-byte aligned");
  if ((int)p->jobs.size() >= kMmPlanJobs)
    return fail(W4A8_E_RANGE, "matmul plan: at most " + std::to_string(kMmPlanJobs) +
                                  " matrices");
  p->jobs.push_back(MmJobSpec{w->d, (int32_t)w->nrows, w->L, w->sh, d_x8, d_y32});
  p->built = false;
  return W4A8_OK;
}

int w4a8_mplan_run(w4a8_mplan *p) {
  if (!p) return fail(W4A8_E_ARG, "null plan");
  if (p->jobs.empty()) return fail(W4A8_E_ARG, "matmul plan has no matrices");
  w4a8_ctx *c = p->ctx;
  DeviceGuard g(c->device);
  const int n = (int)p->jobs.size();
  if (!p->built) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    HIP_TRY(hipStreamIsCapturing(c->stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
      return fail(W4A8_E_ARG, "matmul plan: run it once before capturing it (the first "
                              "run after an add writes its device table)");
    std::vector<uint8_t> host(matmul_job_bytes() * (size_t)n);
    std::vector<int32_t> ns(n);
    HIP_TRY(matmul_plan_prepare(p->jobs.data(), n, p->B, host.data(), &p->cfg, ns.data()));
    for (void *q : {(void *)p->d_table, (void *)p->d_part, p->d_fin})
      if (q) p->retired.push_back(q);
    p->d_table = p->d_fin = nullptr;
    p->d_part = nullptr;
    // a K-split job's slices store their sums to part [ns][B][nrows] int64
    std::vector<size_t> off(n, 0);
    size_t part = 0;
    for (int j = 0; j < n; ++j) {
      if (ns[j] <= 1) continue;
      off[j] = part;
      part += ((size_t)ns[j] * p->B * (size_t)p->jobs[j].nrows * 8 + 255) & ~(size_t)255;
    }
    p->nfin = 0;
    p->fin_max = 0;
    if (part) {
      HIP_TRY(hipMalloc(&p->d_part, part));
      for (int j = 0; j < n; ++j) {
        if (ns[j] <= 1) continue;
        matmul_plan_bind(host.data(), j, (int64_t *)(p->d_part + off[j]));
        const int64_t e = (int64_t)p->B * p->jobs[j].nrows;
        p->fin_max = e > p->fin_max ? e : p->fin_max;
      }
      std::vector<uint8_t> fin(matmul_finish_bytes() * (size_t)n);
      p->nfin = matmul_finish_prepare(host.data(), n, p->B, fin.data());
      HIP_TRY(hipMalloc(&p->d_fin, fin.size()));
      HIP_TRY(hipMemcpy(p->d_fin, fin.data(), fin.size(), hipMemcpyHostToDevice));
    }
    HIP_TRY(hipMalloc(&p->d_table, host.size()));
    HIP_TRY(hipMemcpy(p->d_table, host.data(), host.size(), hipMemcpyHostToDevice));
    p->built = true;
  }
  HIP_TRY(launch_matmul_plan(p->d_table, n, p->cfg, c->d_err, c->stream));
  HIP_TRY(launch_matmul_finish(p->d_fin, p->nfin, p->fin_max, c->d_err, c->stream));
  return W4A8_OK;
}

int w4a8_mplan_destroy(w4a8_mplan *p) {
  if (!p) return W4A8_OK;
  int rc = W4A8_OK;
  for (void *q : {(void *)p->d_table, (void *)p->d_part, p->d_fin})
    if (q) p->retired.push_back(q);
  if (!p->retired.empty()) {
    DeviceGuard g(p->ctx->device);
    bool ok = hipStreamSynchronize(p->ctx->stream) == hipSuccess;
    for (void *q : p->retired) ok = hipFree(q) == hipSuccess && ok;
    if (!ok) rc = fail(W4A8_E_HIP, "matmul plan: freeing its buffers failed");
  }
  delete p;
  return rc;
}

// ------------------------------------------------------------ TOPK-32
// One TOPK-32 launch on the context's stream.  Flags hold the epochs of
// earlier launches; they are cleared (by a kernel, so that a captured graph
// clears them on every replay) when the stream is being captured -- a graph
// replays one fixed epoch -- and before the epoch grows too large.
static int topk_launch(w4a8_ctx *c, const int32_t *d_y, int64_t n, void *lists,
                       int32_t *d_out) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(c->stream, &cs));
  if (cs != hipStreamCaptureStatusNone || c->topk_epoch == 0 ||
      c->topk_epoch + 1 >= kTopkEpochMax) {
    HIP_TRY(launch_fill_i32(c->d_topk_flags, 0, kTopkFlagWords, c->stream));
    c->topk_epoch = 0;
  }
  const int32_t epoch = ++c->topk_epoch;
  HIP_TRY(launch_topk32(d_y, n, lists, c->d_topk_flags, epoch, d_out, c->d_err, c->stream,
                        c->spin_grid));
  // a captured launch replays this epoch with its own clear; the next eager
  // launch clears the flags first
  if (cs != hipStreamCaptureStatusNone) c->topk_epoch = 0;
  return W4A8_OK;
}

// The head's y32 into buf[0, yb), then TOPK-32 with its lists at buf + yb
// (yb = the y32's bytes rounded up to 256).
static int head_topk_launch(w4a8_ctx *c, GemvParams &P, const w4a8_weights *w, uint8_t *buf,
                            int32_t *d_out) {
  const size_t yb = ((size_t)w->nrows * 4 + 255) & ~(size_t)255;
  int32_t *y = (int32_t *)buf;
  P.job[0].epi = EPI_Y32;   // the head's raw y32 (shift 0, seq_format.py:2225-2226)
  P.job[0].out = y;
  HIP_TRY(launch_gemv(P, grid_for(c, P.total_tiles), c->stream));
  return topk_launch(c, y, w->nrows, buf + yb, d_out);
}

int w4a8_head_topk32_async(w4a8_ctx *c, const w4a8_weights *w, int32_t prologue,
                           const void *d_x, const int16_t *d_norm_w, int32_t in_f,
                           int32_t one_plus, int32_t e_x, int32_t *d_out) {
  if (!c || !w || !d_out) return fail(W4A8_E_ARG, "null argument");
  GemvParams P;
  int rc = head_params(c, P, w, prologue, d_x, d_norm_w, in_f, one_plus, e_x);
  if (rc) return rc;
  const size_t yb = ((size_t)w->nrows * 4 + 255) & ~(size_t)255;
  DeviceGuard g(c->device);
  if ((rc = ensure_chain(c, yb + topk_scratch_bytes(w->nrows)))) return rc;
  return head_topk_launch(c, P, w, c->d_chain, d_out);
}

int w4a8_head_topk32_noalloc_async(w4a8_ctx *c, const w4a8_weights *w, int32_t prologue,
                                   const void *d_x, const int16_t *d_norm_w, int32_t in_f,
                                   int32_t one_plus, int32_t e_x, int32_t *d_out) {
  if (!c || !w || !d_out) return fail(W4A8_E_ARG, "null argument");
  const size_t yb = ((size_t)w->nrows * 4 + 255) & ~(size_t)255;
  if (w->nrows > (1 << 18) || yb > kScratchY ||
      topk_scratch_bytes(w->nrows) > kScratchLists)
    return fail(W4A8_E_RANGE, "a head of " + std::to_string(w->nrows) +
                                  " rows exceeds the static scratch's 2^18 rows (" +
                                  std::to_string(kScratchY + kScratchLists) + " bytes)");
  if (!c->d_scratch) return fail(W4A8_E_HIP, "head_topk32_noalloc: no scratch address");
  GemvParams P;
  int rc = head_params(c, P, w, prologue, d_x, d_norm_w, in_f, one_plus, e_x);
  if (rc) return rc;
  DeviceGuard g(c->device);
  return head_topk_launch(c, P, w, c->d_scratch, d_out);
}

int w4a8_topk32(w4a8_ctx *c, const int32_t *y32, int64_t n, int32_t *vals, int32_t *rows,
                int32_t *count, int32_t *overflow) {
  if (!c || !y32 || n < 1) return fail(W4A8_E_ARG, "bad argument");
  if (n > (1 << 18))
    return fail(W4A8_E_RANGE, "topk32: " + std::to_string(n) +
                                  " elements exceed the 18-bit AMAX32 index (2^18)");
  DeviceGuard g(c->device);
  const size_t yb = ((size_t)n * 4 + 255) & ~(size_t)255;
  int rc = ensure_stage(c, yb + 66 * 4);
  if (rc) return rc;
  if ((rc = ensure_chain(c, topk_scratch_bytes(n)))) return rc;
  int32_t *d_y = (int32_t *)c->d_stage, *d_o = (int32_t *)(c->d_stage + yb);
  HIP_TRY(hipMemcpyAsync(d_y, y32, (size_t)n * 4, hipMemcpyHostToDevice, c->stream));
  if ((rc = topk_launch(c, d_y, n, c->d_chain, d_o))) return rc;
  int32_t h[66];
  HIP_TRY(hipMemcpyAsync(h, d_o, sizeof(h), hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  if ((rc = take_err(c))) return rc;
  for (int i = 0; i < 32; ++i) {
    if (vals) vals[i] = h[i];
    if (rows) rows[i] = h[32 + i];
  }
  if (count) *count = h[64];
  if (overflow) *overflow = h[65];
  return W4A8_OK;
}

int w4a8_head_topk32(w4a8_ctx *c, const w4a8_weights *w, int32_t prologue, const void *x,
                     const int16_t *norm_w, int32_t in_f, int32_t one_plus, int32_t *vals,
                     int32_t *rows, int32_t *count, int32_t *overflow) {
  if (!c || !w || !x) return fail(W4A8_E_ARG, "null argument");
  DeviceGuard g(c->device);
  const int32_t K = w->L.K;
  const size_t xb = prologue == PRO_X8 ? (size_t)K : (size_t)K * 2;
  const size_t o_w = (xb + 255) & ~(size_t)255;
  const size_t o_o = o_w + (((size_t)K * 2 + 255) & ~(size_t)255);
  int rc = ensure_stage(c, o_o + 66 * 4);
  if (rc) return rc;
  uint8_t *s = c->d_stage;
  HIP_TRY(hipMemcpyAsync(s, x, xb, hipMemcpyHostToDevice, c->stream));
  if (prologue == PRO_RMSNORM_DYNQ8 && norm_w)
    HIP_TRY(hipMemcpyAsync(s + o_w, norm_w, (size_t)K * 2, hipMemcpyHostToDevice,
                           c->stream));
  rc = w4a8_head_topk32_async(c, w, prologue, s, (const int16_t *)(s + o_w), in_f, one_plus,
                              0, (int32_t *)(s + o_o));
  if (rc) return rc;
  int32_t h[66];
  HIP_TRY(hipMemcpyAsync(h, s + o_o, sizeof(h), hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  if ((rc = take_err(c))) return rc;
  for (int i = 0; i < 32; ++i) {
    if (vals) vals[i] = h[i];
    if (rows) rows[i] = h[32 + i];
  }
  if (count) *count = h[64];
  if (overflow) *overflow = h[65];
  return W4A8_OK;
}

// ------------------------------------------------------------ FFN block
int w4a8_mlp_async(w4a8_ctx *c, const w4a8_weights *gate, const w4a8_weights *up,
                   const w4a8_weights *down, int32_t p0_gate, int32_t p0_up,
                   int32_t p0_down, const int16_t *d_x16, const int16_t *d_norm_w,
                   int32_t in_f, int32_t one_plus, int16_t *d_mlp_out,
                   int16_t *d_res_out) {
  if (!c || !gate || !up || !down || !d_x16) return fail(W4A8_E_ARG, "null argument");
  const int64_t H = gate->L.K, FFN = gate->nrows;
  if (up->L.K != H || up->nrows != FFN || down->L.K != FFN || down->nrows != H)
    return fail(W4A8_E_ARG, "gate and up must be FFN x H and down H x FFN (gate " +
                                std::to_string(gate->nrows) + "x" + std::to_string(H) +
                                ", up " + std::to_string(up->nrows) + "x" +
                                std::to_string(up->L.K) + ", down " +
                                std::to_string(down->nrows) + "x" +
                                std::to_string(down->L.K) + ")");
  if (FFN > 16383)
    return fail(W4A8_E_RANGE, "FFN width " + std::to_string(FFN) +
                                  " does not fit an ALU count (max 16383)");
  if (!d_mlp_out && !d_res_out) return fail(W4A8_E_ARG, "mlp: no output requested");
  // temporaries: sg int16[FFN], u int32[FFN]
  auto al = [](size_t n) { return (n + 255) & ~(size_t)255; };
  const size_t o_u = al(2 * FFN);
  DeviceGuard g(c->device);
  int rc0 = ensure_chain(c, o_u + al(4 * FFN));
  if (rc0) return rc0;
  int16_t *sg = (int16_t *)c->d_chain;
  int32_t *u = (int32_t *)(c->d_chain + o_u);
  // gate and up share the input: one launch, RMSNorm (or not) -> DYNQ8
  const w4a8_weights *gu[2] = {gate, up};
  const int32_t epi_gu[2] = {EPI_SILU32, EPI_MOVY_P32};
  const int32_t p0_gu[2] = {p0_gate, p0_up};
  void *out_gu[2] = {sg, u};
  int rc = site_launch(c, 2, gu, epi_gu, p0_gu, out_gu,
                       d_norm_w ? PRO_RMSNORM_DYNQ8 : PRO_DYNQ8, d_x16, d_norm_w, in_f,
                       one_plus, 0, nullptr, nullptr, nullptr);
  if (rc) return rc;
  // down: EMUL32 at p0 = 12 (gen_layer_script.py:2182-2184) formed in its
  // prologue, then DYNQ8; MOVY int16, and the residual ADD
  // (gen_layer_script.py:1399-1400) in its epilogue
  const int32_t epi_d = EPI_MOVY_I16;
  void *out_d = d_mlp_out ? (void *)d_mlp_out : (void *)d_res_out;
  GemvParams P;
  rc = site_params(c, P, 1, &down, &epi_d, &p0_down, &out_d, PRO_DYNQ8, sg, nullptr, 0, 0,
                   0, nullptr, nullptr, nullptr);
  if (rc) return rc;
  P.job[0].out = d_mlp_out;
  P.pro = PRO_EMUL_DYNQ8;
  P.x2 = u;
  if (d_res_out) {
    P.job[0].epi = EPI_MOVY_I16_ADD;
    P.job[0].res = d_x16;
    P.job[0].res_out = d_res_out;
  }
  HIP_TRY(launch_gemv(P, grid_for(c, P.total_tiles), c->stream));
  return W4A8_OK;
}

// ------------------------------------------------------------------ plans
struct w4a8_plan {
  w4a8_ctx *ctx = nullptr;
  int32_t mode = W4A8_PLAN_GRAPH;
  int32_t fences = W4A8_FENCE_ALL;
  struct Step {
    GemvParams P;
    int grid;
    bool head;
    bool topk;          // a head ending in TOPK-32 (result: 66 int32) instead of the argmax
    int32_t *result;
  };
  std::vector<Step> steps;
  uint64_t *d_partials = nullptr;   // head partial keys (own buffer: graphs pin it)
  int partials_cap = 0;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  hipStream_t exec_stream = nullptr;
  // persistent mode
  GemvParams *d_sites = nullptr;
  uint32_t *d_done = nullptr;
  uint32_t epoch = 0;               // launches since d_done was zeroed
  int8_t *d_stage = nullptr;
  uint64_t *d_stamped = nullptr;    // stamped words of outputs read through them
  int64_t stamped_words = 0;
  std::vector<void *> temps;        // temporaries of the MLP blocks added (w4a8_plan_add_mlp)
  // device buffers of earlier builds (site table, flags, staging, stamped
  // words, head partials): a graph the caller captured from an earlier run
  // still points at them, so they are freed only by destroy
  std::vector<void *> retired;
  // a TOPK-32 head: its rows' y32 (graph mode: int32; persistent: 8-byte
  // stamped words), the scan's lists, and (persistent) the scan's flags
  uint64_t *d_topk_y = nullptr;
  uint8_t *d_topk_lists = nullptr;
  int32_t *d_topk_flags = nullptr;
  bool dependent = false;           // some site waits for, or forms, others' results
  int G = 0;
  int head_site = -1;
  int32_t *head_result = nullptr;
};

static void plan_drop_persistent(w4a8_plan *p) {
  for (void *q : {(void *)p->d_sites, (void *)p->d_done, (void *)p->d_stage,
                  (void *)p->d_stamped})
    if (q) p->retired.push_back(q);
  p->d_sites = nullptr;
  p->d_done = nullptr;
  p->d_stage = nullptr;
  p->d_stamped = nullptr;
  p->stamped_words = 0;
  p->epoch = 0;
  p->G = 0;
}

// Byte ranges a step reads and writes (the weights are read-only for the
// plan's lifetime and never written by a step).
struct ByteRange {
  uintptr_t lo, hi;
};
static void step_ranges(const w4a8_plan::Step &st, std::vector<ByteRange> &rd,
                        std::vector<ByteRange> &wr) {
  const GemvParams &P = st.P;
  auto add = [](std::vector<ByteRange> &v, const void *q, int64_t n) {
    if (q && n > 0) v.push_back({(uintptr_t)q, (uintptr_t)q + (uintptr_t)n});
  };
  add(rd, P.x, P.pro == PRO_X8 ? (int64_t)P.K : 2 * (int64_t)P.K);
  if (P.pro == PRO_RMSNORM_DYNQ8) add(rd, P.norm_w, 2 * (int64_t)P.K);
  if (P.pro == PRO_EMUL_DYNQ8) add(rd, P.x2, 4 * (int64_t)P.K);
  for (int j = 0; j < P.njobs; ++j) {
    const GemvJob &J = P.job[j];
    int64_t es = 0;
    switch (J.epi) {
      case EPI_MOVY_I16:
      case EPI_MOVY_I16_ADD:
      case EPI_SILU32: es = 2; break;
      case EPI_Y32:
      case EPI_MOVY_P32: es = 4; break;
      case EPI_SHIFT_I64: es = 8; break;
      default: es = 0; break;   // EPI_ARGMAX writes the head result below
    }
    add(wr, J.out, es * J.nrows);
    if (J.epi == EPI_MOVY_I16_ADD) {
      add(rd, J.res, 2 * (int64_t)J.nrows);
      add(wr, J.res_out, 2 * (int64_t)J.nrows);
    }
  }
  add(wr, P.x8_out, P.K);
  add(wr, P.e_x_out, 4);
  add(wr, P.xn_out, 2 * (int64_t)P.K);
  if (st.head) add(wr, st.result, (st.topk ? 66 : 2) * (int64_t)sizeof(int32_t));
}
static bool ranges_meet(const std::vector<ByteRange> &a, const std::vector<ByteRange> &b) {
  for (const auto &x : a)
    for (const auto &y : b)
      if (x.lo < y.hi && y.lo < x.hi) return true;
  return false;
}

// The job of site j (since `from`) whose int16 output holds site i's whole x,
// when it is the only write site i's x meets among sites from..i-1 and x
// starts at an even row: (j, job, first word), else j = -1.
struct StampSrc {
  int site = -1, job = -1;   // job kProduct: the site's EMUL32 product words
  int64_t word = 0;
};
constexpr int kProduct = -2;

// Site i forms EMUL32(x2, x) of the two outputs of one site j (since
// `from`): x = job 0's int16 output, x2 = job 1's int32 output, both exactly
// K rows.  When every workgroup holds the same tiles of both jobs (tiles per
// job a multiple of the grid G, at most kPairTiles each), site j can form
// the product itself, and site i reads it through stamped words.
static StampSrc product_source(const std::vector<GemvParams> &sites, int from, int i, int G) {
  StampSrc none, got;
  const GemvParams &C = sites[i];
  if (C.pro != PRO_EMUL_DYNQ8 || C.K % kTileRows || G < 1) return none;
  for (int j = from; j < i; ++j) {
    const GemvParams &P = sites[j];
    if (P.njobs != 2 || P.job[0].out != C.x || (const void *)P.job[1].out != C.x2) continue;
    const int T = C.K / kTileRows;
    if ((P.job[0].epi != EPI_SILU32 && P.job[0].epi != EPI_MOVY_I16) ||
        P.job[1].epi != EPI_MOVY_P32 || P.job[0].nrows != C.K || P.job[1].nrows != C.K ||
        P.total_tiles != 2 * T || T % G || T / G > kPairTiles)
      return none;
    got.site = j;
    got.job = kProduct;
    return got;
  }
  return none;
}
static StampSrc stamp_source(const std::vector<GemvParams> &sites,
                             const std::vector<std::vector<ByteRange>> &wr, int from, int i) {
  StampSrc none, got;
  const GemvParams &C = sites[i];
  if ((C.pro != PRO_DYNQ8 && C.pro != PRO_RMSNORM_DYNQ8) || C.K % 2) return none;
  const ByteRange x{(uintptr_t)C.x, (uintptr_t)C.x + 2 * (uintptr_t)C.K};
  int writers = 0;
  for (int j = from; j < i; ++j)
    for (const auto &w : wr[j])
      if (w.lo < x.hi && x.lo < w.hi) ++writers;
  if (writers != 1) return none;
  for (int j = from; j < i; ++j)
    for (int k = 0; k < sites[j].njobs; ++k) {
      const GemvJob &J = sites[j].job[k];
      if ((J.epi != EPI_MOVY_I16 && J.epi != EPI_SILU32 && J.epi != EPI_MOVY_I16_ADD) ||
          J.nrows % 2)
        continue;
      // a residual ADD's stamped words carry its res_out
      const uintptr_t lo = (uintptr_t)(J.epi == EPI_MOVY_I16_ADD ? (const void *)J.res_out
                                                                  : J.out);
      const uintptr_t hi = lo + 2 * (uintptr_t)J.nrows;
      if (x.lo >= lo && x.hi <= hi && (x.lo - lo) % 4 == 0) {
        got.site = j;
        got.job = k;
        got.word = (int64_t)((x.lo - lo) / 4);
        return got;
      }
    }
  return none;
}

// the persistent launch's grid: one workgroup per CU
static int plan_grid(const w4a8_plan *p) {
  return p->G > 0 ? p->G : p->ctx->num_cu * stream_max_blocks_per_cu();
}

// W4A8_FENCE_AUTO: a site waits only when it reads what a site since the
// last fence writes, or writes what one of those reads or writes -- the
// reference sequencer's FENCE rule (a result is waited for before it is
// consumed, seq_format.py:2077-2231), applied across sites.  When its one
// dependence is reading its int16 input x from one output of such a site,
// it waits for that output's stamped words alone (src[i]); otherwise for
// every workgroup to have finished every earlier site (fence).
static void plan_fences(const w4a8_plan *p, std::vector<GemvParams> &sites,
                        std::vector<StampSrc> &src) {
  const int n = (int)p->steps.size();
  std::vector<std::vector<ByteRange>> rd(n), wr(n);
  for (int i = 0; i < n; ++i) step_ranges(p->steps[i], rd[i], wr[i]);
  src.assign(n, StampSrc{});
  int last = 0;   // first site since the last grid-wide fence
  for (int i = 0; i < n; ++i) {
    bool f = i > 0 && p->fences == W4A8_FENCE_ALL;
    bool meets = false, x_only = true;
    const uintptr_t x0 = (uintptr_t)sites[i].x;
    bool inputs_only = true;   // ... or its x2 (PRO_EMUL_DYNQ8)
    const uintptr_t x2 = (uintptr_t)sites[i].x2;
    for (int j = last; j < i && !f; ++j) {
      for (const auto &a : rd[i])
        if (ranges_meet({a}, wr[j])) {
          meets = true;
          x_only = x_only && a.lo == x0;   // the first read range is x
          inputs_only = inputs_only && (a.lo == x0 || (x2 && a.lo == x2));
        }
      if (ranges_meet(wr[i], rd[j]) || ranges_meet(wr[i], wr[j]))
        meets = true, x_only = inputs_only = false;
    }
    if (meets && !f) {
      if (x_only) src[i] = stamp_source(sites, wr, last, i);
      if (src[i].site < 0 && inputs_only)
        src[i] = product_source(sites, last, i, plan_grid(p));
      f = src[i].site < 0;
    }
    sites[i].fence = f ? 1 : 0;
    if (f) last = i;
    sites[i].fence_at = last;
    sites[i].stamp_src = src[i].site;
    // behind a fence, or reading stamped words, every workgroup computes the
    // site's prologue itself
    sites[i].local_pro = last > 0 || src[i].site >= 0 ? 1 : 0;
  }
}

static int plan_build_persistent(w4a8_plan *p) {
  w4a8_ctx *c = p->ctx;
  const int n = (int)p->steps.size();
  p->head_site = -1;
  for (int i = 0; i < n; ++i)
    if (p->steps[i].head) {
      if (i != n - 1 || p->head_site >= 0)
        return fail(W4A8_E_ARG, "a persistent plan takes one LM head, as its last step");
      p->head_site = i;
      p->head_result = p->steps[i].result;
    }
  p->G = plan_grid(p);
  const bool topk = p->head_site >= 0 && p->steps[p->head_site].topk;
  std::vector<GemvParams> sites(n);
  // tile t of site s goes to workgroup (off_s + t) mod G: the tiles of
  // consecutive sites continue one round-robin, so every workgroup's share
  // of the whole plan differs from the others' by at most one tile
  const int64_t V = (int64_t)p->G;
  int64_t off = 0;
  for (int i = 0; i < n; ++i) {
    sites[i] = p->steps[i].P;
    if (sites[i].pro == PRO_RMSNORM_DYNQ8 && sites[i].K > kStreamNormKMax)
      return fail(W4A8_E_ARG, "a persistent plan takes RMSNorm sites of K <= " +
                                  std::to_string(kStreamNormKMax) + " (step " +
                                  std::to_string(i) + " has K=" +
                                  std::to_string(sites[i].K) + ")");
    sites[i].tile_rot = (int32_t)((V - off % V) % V);
    sites[i].tiles_q = (int32_t)(sites[i].total_tiles / V);
    sites[i].tiles_r = (int32_t)(sites[i].total_tiles % V);
    off += sites[i].total_tiles;
  }
  std::vector<StampSrc> src;
  plan_fences(p, sites, src);
  // stamped words for every output a later site reads through them (one
  // block per (site, job), nrows / 2 words), cleared with the flags
  // (slot kMaxJobs of a site: its EMUL32 product's words)
  std::vector<int64_t> word0(n * (kMaxJobs + 1), -1);
  auto slot = [&](const StampSrc &a) { return a.site * (kMaxJobs + 1) +
                                              (a.job == kProduct ? kMaxJobs : a.job); };
  int64_t words = 0;
  for (int i = 0; i < n; ++i)
    if (src[i].site >= 0) {
      int64_t &w0 = word0[slot(src[i])];
      if (w0 < 0) {
        w0 = words;
        words += (src[i].job == kProduct ? sites[i].K : sites[src[i].site].job[src[i].job].nrows) / 2;
      }
    }
  HIP_TRY(hipMalloc(&p->d_sites, sizeof(GemvParams) * (size_t)n));
  HIP_TRY(hipMalloc(&p->d_done, sizeof(uint32_t) * stream_counter_words(p->G, n)));
  HIP_TRY(hipMalloc(&p->d_stage, (size_t)kStageBytes * (size_t)n));
  p->stamped_words = words;
  p->dependent = false;
  for (int i = 0; i < n; ++i)
    p->dependent = p->dependent || sites[i].local_pro || sites[i].stamp_src >= 0 ||
                   sites[i].pro == PRO_EMUL_DYNQ8;
  if (words > 0) HIP_TRY(hipMalloc(&p->d_stamped, sizeof(uint64_t) * (size_t)words));
  for (int i = 0; i < n; ++i) {
    for (int k = 0; k < sites[i].njobs; ++k) {
      const int64_t w0 = word0[i * (kMaxJobs + 1) + k];
      sites[i].job[k].stamped = w0 >= 0 ? p->d_stamped + w0 : nullptr;
    }
    const int64_t pw0 = word0[i * (kMaxJobs + 1) + kMaxJobs];
    sites[i].prod_stamped = pw0 >= 0 ? p->d_stamped + pw0 : nullptr;
    sites[i].x_stamped = src[i].site >= 0 ? p->d_stamped + word0[slot(src[i])] + src[i].word
                                          : nullptr;
    // a site reading a product formed by its producer is a DYNQ8 site of it
    if (src[i].job == kProduct) sites[i].pro = PRO_DYNQ8;
    // the TOPK-32 head's rows go out as stamped words, for the scan that runs
    // in the same launch
    if (topk && i == p->head_site) {
      sites[i].job[0].epi = EPI_TOPK;
      sites[i].job[0].out = p->d_topk_y;
    }
    // stream_kernel's residual ADD: an EPI_MOVY_I16 job with res_out set
    for (int k = 0; k < sites[i].njobs; ++k) {
      GemvJob &J = sites[i].job[k];
      if (J.epi == EPI_MOVY_I16_ADD) J.epi = EPI_MOVY_I16;
      else J.res_out = nullptr;
    }
  }
  if (topk && !p->d_topk_flags)
    HIP_TRY(hipMalloc(&p->d_topk_flags, sizeof(int32_t) * kTopkFlagWords));
  p->epoch = 0;
  HIP_TRY(hipMemcpy(p->d_sites, sites.data(), sizeof(GemvParams) * (size_t)n,
                    hipMemcpyHostToDevice));
  return W4A8_OK;
}

static int plan_launch_persistent(w4a8_plan *p, hipStream_t s, hipEvent_t e0,
                                  hipEvent_t e1, uint64_t *trace = nullptr) {
  const int n = (int)p->steps.size();
  // The flag words are zeroed once, not per launch: each launch's flag values
  // exceed the previous launch's (they grow by n + 1 per launch), and the
  // head's words are left zero by the launch that used them.  They are zeroed
  // again before the values would pass 2^32, and in every launch a graph
  // captures (each replay of the graph stores the same values).
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(s, &cs));
  const bool topk = p->head_site >= 0 && p->steps[p->head_site].topk;
  const int64_t topk_rows = topk ? p->steps[p->head_site].P.job[0].nrows : 0;
  // (the TOPK-32 scan's flags hold 2 epoch + 1 in an int32)
  if (p->epoch == 0 || cs != hipStreamCaptureStatusNone ||
      (uint64_t)(p->epoch + 1) * (uint64_t)(n + 1) > 0xFFFFFFFFull ||
      (topk && p->epoch + 1 >= (uint32_t)kTopkEpochMax)) {
    HIP_TRY(launch_fill_i32((int32_t *)p->d_done, 0, (int64_t)stream_counter_words(p->G, n), s));
    if (p->stamped_words > 0)
      HIP_TRY(launch_fill_i32((int32_t *)p->d_stamped, 0, 2 * p->stamped_words, s));
    if (topk) {
      HIP_TRY(launch_fill_i32(p->d_topk_flags, 0, kTopkFlagWords, s));
      HIP_TRY(launch_fill_i32((int32_t *)p->d_topk_y, 0, 2 * topk_rows, s));
    }
    p->epoch = 0;
  }
  StreamParams sp{};
  sp.sites = p->d_sites;
  sp.nsites = (int32_t)n;
  sp.head_site = topk ? -1 : p->head_site;
  if (topk) {
    sp.topk_y = p->d_topk_y;
    sp.topk_lists = (uint64_t *)p->d_topk_lists;
    sp.topk_flags = p->d_topk_flags;
    sp.topk_out = p->head_result;
    sp.topk_rows = (int32_t)topk_rows;
  }
  sp.done = p->d_done;
  sp.epoch = ++p->epoch;
  sp.stage = p->d_stage;
  sp.err = p->ctx->d_err;
  sp.result = p->head_result;
  sp.trace = trace;
  sp.grid_spin = p->ctx->spin_grid;
  sp.lds_spin = p->ctx->spin_lds;
  HIP_TRY(launch_stream(sp, p->G, s, p->mode == W4A8_PLAN_PERSISTENT_COOP, p->dependent, e0,
                        e1));
  // A captured launch replays this epoch with its own fill; the memory holds
  // whatever ran last, so the next eager launch clears it first.
  if (cs != hipStreamCaptureStatusNone) p->epoch = 0;
  return W4A8_OK;
}

static void plan_drop_graph(w4a8_plan *p) {
  if (p->exec) (void)hipGraphExecDestroy(p->exec);
  if (p->graph) (void)hipGraphDestroy(p->graph);
  p->exec = nullptr;
  p->graph = nullptr;
  plan_drop_persistent(p);
}

static int plan_enqueue(w4a8_plan *p, hipStream_t s) {
  for (auto &st : p->steps) {
    if (st.topk) {
      // the head's raw y32 (shift 0, seq_format.py:2225-2226), then the scan
      GemvParams P = st.P;
      P.job[0].epi = EPI_Y32;
      P.job[0].out = p->d_topk_y;
      HIP_TRY(launch_gemv(P, st.grid, s));
      int rc = topk_launch(p->ctx, (const int32_t *)p->d_topk_y, P.job[0].nrows,
                           p->d_topk_lists, st.result);
      if (rc) return rc;
      continue;
    }
    HIP_TRY(launch_gemv(st.P, st.grid, s));
    if (st.head) HIP_TRY(launch_argmax_final(st.P.partials, st.grid, st.result, s));
  }
  return W4A8_OK;
}

int w4a8_plan_create(w4a8_ctx *c, w4a8_plan **out) {
  if (!c || !out) return fail(W4A8_E_ARG, "null argument");
  *out = new w4a8_plan();
  (*out)->ctx = c;
  return W4A8_OK;
}

int w4a8_plan_add_site(w4a8_plan *p, int32_t nmat, const w4a8_weights *const *w,
                       const int32_t *epilogue, const int32_t *p0, void *const *d_out,
                       int32_t prologue, const void *d_x, const int16_t *d_norm_w,
                       int32_t in_f, int32_t one_plus, int32_t e_x, int8_t *d_x8_out,
                       int32_t *d_e_x_out, int16_t *d_xn_out) {
  if (!p || !w || !epilogue || !p0 || !d_out) return fail(W4A8_E_ARG, "null argument");
  w4a8_plan::Step st{};
  int rc = site_params(p->ctx, st.P, nmat, w, epilogue, p0, d_out, prologue, d_x,
                       d_norm_w, in_f, one_plus, e_x, d_x8_out, d_e_x_out, d_xn_out);
  if (rc) return rc;
  st.grid = grid_for(p->ctx, st.P.total_tiles);
  st.head = false;
  st.result = nullptr;
  p->steps.push_back(st);
  plan_drop_graph(p);
  return W4A8_OK;
}

int w4a8_plan_add_site_emul(w4a8_plan *p, int32_t nmat, const w4a8_weights *const *w,
                            const int32_t *epilogue, const int32_t *p0, void *const *d_out,
                            const int16_t *d_x, const int32_t *d_x2, int8_t *d_x8_out,
                            int32_t *d_e_x_out) {
  if (!p || !w || !epilogue || !p0 || !d_out) return fail(W4A8_E_ARG, "null argument");
  if (!d_x2 || !aligned16(d_x2)) return fail(W4A8_E_ARG, "x2 must be a 16-byte aligned pointer");
  w4a8_plan::Step st{};
  int rc = site_params(p->ctx, st.P, nmat, w, epilogue, p0, d_out, PRO_DYNQ8, d_x, nullptr, 0,
                       0, 0, d_x8_out, d_e_x_out, nullptr);
  if (rc) return rc;
  st.P.pro = PRO_EMUL_DYNQ8;
  st.P.x2 = d_x2;
  st.grid = grid_for(p->ctx, st.P.total_tiles);
  st.head = false;
  st.result = nullptr;
  p->steps.push_back(st);
  plan_drop_graph(p);
  return W4A8_OK;
}

int w4a8_plan_add_site_emul_res(w4a8_plan *p, const w4a8_weights *down, int32_t p0,
                                int16_t *d_out, const int16_t *d_x, const int32_t *d_x2,
                                const int16_t *d_res, int16_t *d_res_out) {
  if (!p || !down || !d_res || !d_res_out) return fail(W4A8_E_ARG, "null argument");
  if (!d_x2 || !aligned16(d_x2)) return fail(W4A8_E_ARG, "x2 must be a 16-byte aligned pointer");
  w4a8_plan::Step st{};
  const int32_t epi = EPI_MOVY_I16;
  void *out = d_res_out;
  int rc = site_params(p->ctx, st.P, 1, &down, &epi, &p0, &out, PRO_DYNQ8, d_x, nullptr, 0, 0,
                       0, nullptr, nullptr, nullptr);
  if (rc) return rc;
  st.P.pro = PRO_EMUL_DYNQ8;
  st.P.x2 = d_x2;
  st.P.job[0].epi = EPI_MOVY_I16_ADD;
  st.P.job[0].out = d_out;
  st.P.job[0].res = d_res;
  st.P.job[0].res_out = d_res_out;
  st.grid = grid_for(p->ctx, st.P.total_tiles);
  st.head = false;
  st.result = nullptr;
  p->steps.push_back(st);
  plan_drop_graph(p);
  return W4A8_OK;
}

int w4a8_plan_add_mlp(w4a8_plan *p, const w4a8_weights *gate, const w4a8_weights *up,
                      const w4a8_weights *down, int32_t p0_gate, int32_t p0_up,
                      int32_t p0_down, const int16_t *d_x16, const int16_t *d_norm_w,
                      int32_t in_f, int32_t one_plus, int16_t *d_mlp_out, int16_t *d_res_out) {
  if (!p || !gate || !up || !down || !d_x16) return fail(W4A8_E_ARG, "null argument");
  const int64_t H = gate->L.K, FFN = gate->nrows;
  if (up->L.K != H || up->nrows != FFN || down->L.K != FFN || down->nrows != H)
    return fail(W4A8_E_ARG, "gate and up must be FFN x H and down H x FFN");
  if (!d_mlp_out && !d_res_out) return fail(W4A8_E_ARG, "mlp: no output requested");
  // the layer's temporaries, owned by the plan: sg int16[FFN], u int32[FFN]
  DeviceGuard g(p->ctx->device);
  uint8_t *tmp = nullptr;
  const size_t o_u = ((size_t)2 * FFN + 255) & ~(size_t)255;
  HIP_TRY(hipMalloc(&tmp, o_u + (size_t)4 * FFN));
  p->temps.push_back(tmp);
  int16_t *sg = (int16_t *)tmp;
  int32_t *u = (int32_t *)(tmp + o_u);
  const w4a8_weights *gu[2] = {gate, up};
  const int32_t epi_gu[2] = {EPI_SILU32, EPI_MOVY_P32};
  const int32_t p0_gu[2] = {p0_gate, p0_up};
  void *out_gu[2] = {sg, u};
  // the block goes in whole or not at all: a failed add takes back what
  // the block added before it, so the plan's steps stay the caller's sites
  const size_t n0 = p->steps.size();
  auto undo = [&](int rc) {
    if (p->steps.size() != n0) {
      p->steps.resize(n0);
      plan_drop_graph(p);
    }
    p->temps.pop_back();
    (void)hipFree(tmp);
    return rc;
  };
  int rc = w4a8_plan_add_site(p, 2, gu, epi_gu, p0_gu, out_gu,
                              d_norm_w ? PRO_RMSNORM_DYNQ8 : PRO_DYNQ8, d_x16, d_norm_w, in_f,
                              one_plus, 0, nullptr, nullptr, nullptr);
  if (rc) return undo(rc);
  if (!d_res_out) {
    const int32_t epi = EPI_MOVY_I16;
    void *out = d_mlp_out;
    rc = w4a8_plan_add_site_emul(p, 1, &down, &epi, &p0_down, &out, sg, u, nullptr, nullptr);
  } else {
    rc = w4a8_plan_add_site_emul_res(p, down, p0_down, d_mlp_out, sg, u, d_x16, d_res_out);
  }
  return rc ? undo(rc) : W4A8_OK;
}

int w4a8_plan_add_head(w4a8_plan *p, const w4a8_weights *w, int32_t prologue,
                       const void *d_x, const int16_t *d_norm_w, int32_t in_f,
                       int32_t one_plus, int32_t e_x, int32_t *d_result) {
  if (!p || !d_result) return fail(W4A8_E_ARG, "null argument");
  w4a8_plan::Step st{};
  int rc = head_params(p->ctx, st.P, w, prologue, d_x, d_norm_w, in_f, one_plus, e_x);
  if (rc) return rc;
  st.grid = grid_for(p->ctx, st.P.total_tiles);
  st.head = true;
  st.result = d_result;
  // every head of the plan gets its own slice of the partials buffer
  int used = 0;
  for (auto &o : p->steps) if (o.head) used += o.grid;
  if (used + st.grid > p->partials_cap) {
    DeviceGuard g(p->ctx->device);
    const int cap = (used + st.grid) * 2;
    uint64_t *np_ = nullptr;
    HIP_TRY(hipMalloc(&np_, sizeof(uint64_t) * (size_t)cap));
    if (p->d_partials) p->retired.push_back(p->d_partials);
    p->d_partials = np_;
    p->partials_cap = cap;
    int off = 0;
    for (auto &o : p->steps)
      if (o.head) { o.P.partials = p->d_partials + off; off += o.grid; }
  }
  st.P.partials = p->d_partials + used;
  p->steps.push_back(st);
  plan_drop_graph(p);
  return W4A8_OK;
}

int w4a8_plan_add_head_topk32(w4a8_plan *p, const w4a8_weights *w, int32_t prologue,
                              const void *d_x, const int16_t *d_norm_w, int32_t in_f,
                              int32_t one_plus, int32_t e_x, int32_t *d_out) {
  if (!p || !d_out) return fail(W4A8_E_ARG, "null argument");
  for (auto &o : p->steps)
    if (o.topk) return fail(W4A8_E_ARG, "a plan takes one TOPK-32 head");
  w4a8_plan::Step st{};
  int rc = head_params(p->ctx, st.P, w, prologue, d_x, d_norm_w, in_f, one_plus, e_x);
  if (rc) return rc;
  DeviceGuard g(p->ctx->device);
  // y32 of every row: int32 in graph mode, 8-byte stamped words in a
  // persistent launch; the scan's lists (the plan's own, so that graphs of
  // it hold them)
  const size_t yb = ((size_t)w->nrows * 8 + 255) & ~(size_t)255;
  uint8_t *buf = nullptr;
  HIP_TRY(hipMalloc(&buf, yb + topk_scratch_bytes(w->nrows)));
  HIP_TRY(hipMemset(buf, 0, yb));
  if (p->d_topk_y) p->retired.push_back(p->d_topk_y);
  p->d_topk_y = (uint64_t *)buf;
  p->d_topk_lists = buf + yb;
  st.P.job[0].epi = EPI_Y32;
  st.P.job[0].out = p->d_topk_y;
  st.grid = grid_for(p->ctx, st.P.total_tiles);
  st.head = true;
  st.topk = true;
  st.result = d_out;
  p->steps.push_back(st);
  plan_drop_graph(p);
  return W4A8_OK;
}

int w4a8_plan_set_mode(w4a8_plan *p, int32_t mode) {
  if (!p || (mode != W4A8_PLAN_GRAPH && mode != W4A8_PLAN_PERSISTENT &&
             mode != W4A8_PLAN_PERSISTENT_COOP))
    return fail(W4A8_E_ARG, "unknown plan mode");
  if (mode != p->mode) plan_drop_graph(p);
  p->mode = mode;
  return W4A8_OK;
}

int w4a8_plan_set_fences(w4a8_plan *p, int32_t fences) {
  if (!p || (fences != W4A8_FENCE_ALL && fences != W4A8_FENCE_AUTO))
    return fail(W4A8_E_ARG, "unknown fence mode");
  if (fences != p->fences) plan_drop_graph(p);
  p->fences = fences;
  return W4A8_OK;
}

int w4a8_plan_fences(w4a8_plan *p, int32_t n, int32_t *fenced) {
  if (!p || (n > 0 && !fenced)) return fail(W4A8_E_ARG, "null argument");
  if (n != (int32_t)p->steps.size())
    return fail(W4A8_E_ARG, "plan has " + std::to_string(p->steps.size()) + " steps");
  std::vector<GemvParams> sites(n);
  for (int i = 0; i < n; ++i) sites[i] = p->steps[i].P;
  std::vector<StampSrc> src;
  plan_fences(p, sites, src);
  for (int i = 0; i < n; ++i) fenced[i] = sites[i].fence ? 1 : (src[i].site >= 0 ? 2 : 0);
  return W4A8_OK;
}

int w4a8_plan_run(w4a8_plan *p) {
  if (!p) return fail(W4A8_E_ARG, "null plan");
  if (p->steps.empty()) return W4A8_OK;
  w4a8_ctx *c = p->ctx;
  DeviceGuard g(c->device);
  if (p->mode != W4A8_PLAN_GRAPH) {
    if (!p->d_sites) {
      int rc = plan_build_persistent(p);
      if (rc) {
        plan_drop_persistent(p);
        return rc;
      }
    }
    return plan_launch_persistent(p, c->stream, nullptr, nullptr);
  }
  if (p->exec && p->exec_stream != c->stream) plan_drop_graph(p);
  if (!p->exec) {
    HIP_TRY(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    int rc = plan_enqueue(p, c->stream);
    hipGraph_t gr = nullptr;
    hipError_t e = hipStreamEndCapture(c->stream, &gr);
    if (rc) {
      if (gr) (void)hipGraphDestroy(gr);
      return rc;
    }
    if (e != hipSuccess)
      return fail(W4A8_E_HIP, std::string("hipStreamEndCapture: ") + hipGetErrorString(e));
    p->graph = gr;
    HIP_TRY(hipGraphInstantiate(&p->exec, p->graph, nullptr, nullptr, 0));
    p->exec_stream = c->stream;
  }
  HIP_TRY(hipGraphLaunch(p->exec, c->stream));
  return W4A8_OK;
}

int w4a8_plan_profile(w4a8_plan *p, int32_t n, float *ms) {
  if (!p || (n > 0 && !ms)) return fail(W4A8_E_ARG, "null argument");
  if (n != (int32_t)p->steps.size())
    return fail(W4A8_E_ARG, "plan has " + std::to_string(p->steps.size()) + " steps");
  w4a8_ctx *c = p->ctx;
  DeviceGuard g(c->device);
  if (p->mode != W4A8_PLAN_GRAPH) {
    // one launch runs every step: its per-site times come from the
    // wall-clock stamps workgroup 0 takes as it starts each site, scaled so
    // that they sum to the launch's event-measured time
    if (!p->d_sites) {
      int rc = plan_build_persistent(p);
      if (rc) return rc;
    }
    uint64_t *d_trace = nullptr;
    HIP_TRY(hipMalloc(&d_trace, sizeof(uint64_t) * (size_t)(n + 1)));
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = W4A8_OK;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)
      rc = fail(W4A8_E_HIP, "hipEventCreate");
    if (!rc) rc = plan_launch_persistent(p, c->stream, e0, e1, d_trace);
    if (!rc && hipStreamSynchronize(c->stream) != hipSuccess) rc = fail(W4A8_E_HIP, "sync");
    std::vector<uint64_t> tr(n + 1);
    float total = 0.f;
    if (!rc && (hipEventElapsedTime(&total, e0, e1) != hipSuccess ||
                hipMemcpy(tr.data(), d_trace, sizeof(uint64_t) * (n + 1),
                          hipMemcpyDeviceToHost) != hipSuccess))
      rc = fail(W4A8_E_HIP, "profile readback");
    if (!rc) {
      const double span = (double)(tr[n] - tr[0]);
      for (int i = 0; i < n; ++i)
        ms[i] = span > 0 ? (float)(total * (double)(tr[i + 1] - tr[i]) / span) : 0.f;
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipFree(d_trace);
    return rc;
  }
  std::vector<hipEvent_t> ev(2 * p->steps.size(), nullptr);
  int rc = W4A8_OK;
  for (auto &e : ev)
    if (hipEventCreate(&e) != hipSuccess) rc = fail(W4A8_E_HIP, "hipEventCreate");
  for (size_t i = 0; !rc && i < p->steps.size(); ++i) {
    auto &st = p->steps[i];
    if (st.topk) {
      // the head's y32 (st.P: EPI_Y32 into the plan's buffer), then its scan;
      // the step's time covers both
      hipError_t e = launch_gemv_timed(st.P, st.grid, c->stream, ev[2 * i], nullptr);
      if (e != hipSuccess) {
        rc = fail(W4A8_E_HIP, hipGetErrorString(e));
        break;
      }
      rc = topk_launch(c, (const int32_t *)p->d_topk_y, st.P.job[0].nrows, p->d_topk_lists,
                       st.result);
      if (!rc && hipEventRecord(ev[2 * i + 1], c->stream) != hipSuccess)
        rc = fail(W4A8_E_HIP, "hipEventRecord");
      continue;
    }
    hipError_t e = launch_gemv_timed(st.P, st.grid, c->stream, ev[2 * i], ev[2 * i + 1]);
    if (e == hipSuccess && st.head)
      e = launch_argmax_final(st.P.partials, st.grid, st.result, c->stream);
    if (e != hipSuccess) rc = fail(W4A8_E_HIP, hipGetErrorString(e));
  }
  if (!rc && hipStreamSynchronize(c->stream) != hipSuccess) rc = fail(W4A8_E_HIP, "sync");
  for (size_t i = 0; !rc && i < p->steps.size(); ++i)
    if (hipEventElapsedTime(&ms[i], ev[2 * i], ev[2 * i + 1]) != hipSuccess)
      rc = fail(W4A8_E_HIP, "hipEventElapsedTime");
  for (auto &e : ev)
    if (e) (void)hipEventDestroy(e);
  return rc;
}

int w4a8_plan_time_launches(w4a8_plan *p, int32_t n, float *ms) {
  if (!p || n < 1 || !ms) return fail(W4A8_E_ARG, "null argument or n < 1");
  if (p->mode == W4A8_PLAN_GRAPH)
    return fail(W4A8_E_ARG, "w4a8_plan_time_launches times persistent plans");
  if (p->steps.empty()) return fail(W4A8_E_ARG, "empty plan");
  w4a8_ctx *c = p->ctx;
  DeviceGuard g(c->device);
  if (!p->d_sites) {
    int rc = plan_build_persistent(p);
    if (rc) {
      plan_drop_persistent(p);
      return rc;
    }
  }
  std::vector<hipEvent_t> ev(2 * (size_t)n, nullptr);
  int rc = W4A8_OK;
  for (auto &e : ev)
    if (!rc && hipEventCreate(&e) != hipSuccess) rc = fail(W4A8_E_HIP, "hipEventCreate");
  for (int i = 0; !rc && i < n; ++i)
    rc = plan_launch_persistent(p, c->stream, ev[2 * i], ev[2 * i + 1]);
  if (!rc && hipStreamSynchronize(c->stream) != hipSuccess) rc = fail(W4A8_E_HIP, "sync");
  for (int i = 0; !rc && i < n; ++i)
    if (hipEventElapsedTime(&ms[i], ev[2 * i], ev[2 * i + 1]) != hipSuccess)
      rc = fail(W4A8_E_HIP, "hipEventElapsedTime");
  for (auto &e : ev)
    if (e) (void)hipEventDestroy(e);
  return rc ? rc : take_err(c);
}

int w4a8_plan_destroy(w4a8_plan *p) {
  if (!p) return W4A8_OK;
  DeviceGuard g(p->ctx->device);
  (void)hipStreamSynchronize(p->ctx->stream);
  plan_drop_graph(p);
  if (p->d_partials) (void)hipFree(p->d_partials);
  for (void *t : p->temps) (void)hipFree(t);
  for (void *q : p->retired) (void)hipFree(q);
  if (p->d_topk_y) (void)hipFree(p->d_topk_y);
  if (p->d_topk_flags) (void)hipFree(p->d_topk_flags);
  delete p;
  return W4A8_OK;
}

}  // extern "C"
