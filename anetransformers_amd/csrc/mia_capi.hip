// mia_capi.hip -- extern "C" shim of libmiattn.so (see include/miattn.h).
// Host code only: validation, per-device context (stream, split-K scratch,
// work buffers) and launch planning.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/miattn.h"
#include "../../include/mia_peaks.h"
#include "mia_kernels.h"

// Scratch of mia_decode_step_noalloc, one copy per device for the life of the
// process: the split-K partials (m, l, o) of one decode call, up to 256 chunks
// x 8 kv heads x 4 query heads x (128 + 2) floats.  Host code never uses this
// name as an address: mia_init takes each device's address of it once
// (hipGetSymbolAddress) into DevCtx::noalloc.
constexpr size_t kNoAllocScratchBytes = 4259840;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 16;
constexpr int kG = 4;
constexpr int kHD = 128;
constexpr int kMaxSeq = 1 << 22;  // ring capacity limit; in-layer offsets are 64-bit in every kernel
// mia_attention_chunk: up to this many tokens, each finds out whether a later
// token takes its slot by scanning them (S^2 / 2 reads); longer chunks use a
// per-slot area instead (one more launch, linear in S).
constexpr int kChunkScanMax = 64;
// The fp16 GEMMs of the weight types other than Q4_0 (hipBLASLt): workspace
// size, algorithms timed on a shape's first call, shapes remembered.
constexpr size_t kLtWorkspace = size_t(64) << 20;
constexpr int kLtCandidates = 4;
constexpr size_t kLtMaxShapes = 64;

struct LtPick {
  int m, n, k;
  hipblasLtMatmulAlgo_t algo;
};

struct DevCtx {
  bool ready = false;
  hipStream_t stream = nullptr;
  int num_cus = 256;
  void *split = nullptr;  // split-K partials (allocated on demand)
  size_t split_bytes = 0;
  // The address of this device's copy of `scratch` (below), for
  // mia_decode_step_noalloc; taken once by mia_init.
  void *noalloc = nullptr;
  void *work = nullptr;  // fp16 draft staging for mia_attention_step
  size_t work_bytes = 0;
  void *layer_work = nullptr;  // activations of mia_prefill_layer
  size_t layer_work_bytes = 0;
  void *gemm_work = nullptr;  // split-K partial products of the Q4_0 GEMM
  size_t gemm_work_bytes = 0;
  void *split_work = nullptr;  // the Q4_0 GEMM's activations as fp16 hi and lo planes
  size_t split_work_bytes = 0;
  int *owner = nullptr;  // long chunks of mia_attention_chunk: last token per ring slot, -1 at rest
  int owner_slots = 0;
  // Weight types other than Q4_0 in the GEMM: the weights' fp16 planes and
  // the partial products, multiplied by hipBLASLt (handle and workspace
  // created on first use, the algorithm of each GEMM shape picked on its
  // first call: lt_gemm).
  float *wbuf = nullptr;
  size_t wbuf_bytes = 0;
  hipblasLtHandle_t lt = nullptr;
  void *lt_ws = nullptr;
  std::vector<LtPick> lt_picks;
  void *dl_work = nullptr;  // mia_decode_layer's vectors
  size_t dl_work_bytes = 0;
  // Opt-in kernel timing: an event pair around the main kernel of each call
  // (kind 0 = decode kernel, 1 = flash kernel, 2 = Q4_0 matvec kernel,
  // 3 = Q4_0 GEMM kernel, 4 = the empty kernel of mia_peak_empty, 5 = the
  // matvec kernel of the other weight types).
  bool prof_on = false;
  std::vector<hipEvent_t> prof_ev[6];
  size_t prof_n[6] = {0, 0, 0, 0, 0, 0};
};

DevCtx g_ctx[kMaxDevices];
std::mutex g_mu;
thread_local char g_err[512] = "";

int set_err(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

#define HIP_TRY(call)                                                                    \
  do {                                                                                   \
    hipError_t e_ = (call);                                                              \
    if (e_ != hipSuccess)                                                                \
      return set_err(MIA_ERR_HIP, "%s failed: %s", #call, hipGetErrorString(e_));       \
  } while (0)

int current_ctx(DevCtx **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_err(MIA_ERR_NO_DEVICE, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return set_err(MIA_ERR_NO_DEVICE, "device %d out of range", dev);
  if (!g_ctx[dev].ready) {
    int rc = mia_init(dev);
    if (rc) return rc;
  }
  *out = &g_ctx[dev];
  return MIA_OK;
}

hipStream_t pick_stream(DevCtx *c, void *stream) {
  return stream ? reinterpret_cast<hipStream_t>(stream) : c->stream;
}

// Grows the split-K scratch.  Growth synchronises the device so that no
// queued kernel still uses the old buffer.
int ensure_scratch(DevCtx *c, size_t bytes) {
  if (bytes > c->split_bytes) {
    HIP_TRY(hipDeviceSynchronize());
    if (c->split) HIP_TRY(hipFree(c->split));
    c->split = nullptr;
    c->split_bytes = 0;
    size_t sz = bytes + (bytes >> 2);
    HIP_TRY(hipMalloc(&c->split, sz));
    c->split_bytes = sz;
  }
  return MIA_OK;
}

int ensure_work(DevCtx *c, size_t bytes) {
  if (bytes > c->work_bytes) {
    HIP_TRY(hipDeviceSynchronize());
    if (c->work) HIP_TRY(hipFree(c->work));
    c->work = nullptr;
    c->work_bytes = 0;
    HIP_TRY(hipMalloc(&c->work, bytes));
    c->work_bytes = bytes;
  }
  return MIA_OK;
}

int ensure_owner(DevCtx *c, int slots) {
  if (slots > c->owner_slots) {
    HIP_TRY(hipDeviceSynchronize());
    if (c->owner) HIP_TRY(hipFree(c->owner));
    c->owner = nullptr;
    c->owner_slots = 0;
    HIP_TRY(hipMalloc((void **)&c->owner, (size_t)slots * sizeof(int)));
    HIP_TRY(hipMemset(c->owner, 0xFF, (size_t)slots * sizeof(int)));  // -1 everywhere
    c->owner_slots = slots;
  }
  return MIA_OK;
}

int ensure_layer_work(DevCtx *c, size_t bytes) {
  if (bytes > c->layer_work_bytes) {
    HIP_TRY(hipDeviceSynchronize());
    if (c->layer_work) HIP_TRY(hipFree(c->layer_work));
    c->layer_work = nullptr;
    c->layer_work_bytes = 0;
    HIP_TRY(hipMalloc(&c->layer_work, bytes));
    c->layer_work_bytes = bytes;
  }
  return MIA_OK;
}

int ensure_split_work(DevCtx *c, size_t bytes) {
  if (bytes > c->split_work_bytes) {
    HIP_TRY(hipDeviceSynchronize());
    if (c->split_work) HIP_TRY(hipFree(c->split_work));
    c->split_work = nullptr;
    c->split_work_bytes = 0;
    HIP_TRY(hipMalloc(&c->split_work, bytes));
    c->split_work_bytes = bytes;
  }
  return MIA_OK;
}

int ensure_gemm_work(DevCtx *c, size_t bytes) {
  if (bytes > c->gemm_work_bytes) {
    HIP_TRY(hipDeviceSynchronize());
    if (c->gemm_work) HIP_TRY(hipFree(c->gemm_work));
    c->gemm_work = nullptr;
    c->gemm_work_bytes = 0;
    HIP_TRY(hipMalloc(&c->gemm_work, bytes));
    c->gemm_work_bytes = bytes;
  }
  return MIA_OK;
}

int ensure_wbuf(DevCtx *c, size_t bytes) {
  if (bytes > c->wbuf_bytes) {
    HIP_TRY(hipDeviceSynchronize());
    if (c->wbuf) HIP_TRY(hipFree(c->wbuf));
    c->wbuf = nullptr;
    c->wbuf_bytes = 0;
    HIP_TRY(hipMalloc((void **)&c->wbuf, bytes));
    c->wbuf_bytes = bytes;
  }
  return MIA_OK;
}

int ensure_dl_work(DevCtx *c, size_t bytes) {
  if (bytes > c->dl_work_bytes) {
    HIP_TRY(hipDeviceSynchronize());
    if (c->dl_work) HIP_TRY(hipFree(c->dl_work));
    c->dl_work = nullptr;
    c->dl_work_bytes = 0;
    HIP_TRY(hipMalloc(&c->dl_work, bytes));
    c->dl_work_bytes = bytes;
  }
  return MIA_OK;
}

int ensure_lt(DevCtx *c) {
  if (c->lt_ws == nullptr) HIP_TRY(hipMalloc(&c->lt_ws, kLtWorkspace));
  if (c->lt == nullptr) {
    hipblasLtHandle_t h = nullptr;
    const hipblasStatus_t st = hipblasLtCreate(&h);
    if (st != HIPBLAS_STATUS_SUCCESS) return set_err(MIA_ERR_HIP, "hipblasLtCreate: status %d", (int)st);
    c->lt = h;
  }
  return MIA_OK;
}

// The descriptors of C = A^T B: A the fp16 weights (column-major k x m, i.e.
// m rows of k values), B the fp16 activations (k x n: n rows of k), C fp32
// column-major m x n (n rows of m outputs), fp32 accumulation.
struct LtDesc {
  hipblasLtMatmulDesc_t md = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasStatus_t st = HIPBLAS_STATUS_SUCCESS;
  LtDesc(int m, int n, int k) {
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    st = hipblasLtMatmulDescCreate(&md, HIPBLAS_COMPUTE_32F, HIP_R_32F);
    if (st == HIPBLAS_STATUS_SUCCESS)
      st = hipblasLtMatmulDescSetAttribute(md, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta));
    if (st == HIPBLAS_STATUS_SUCCESS)
      st = hipblasLtMatmulDescSetAttribute(md, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb));
    if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatrixLayoutCreate(&la, HIP_R_16F, k, m, k);
    if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatrixLayoutCreate(&lb, HIP_R_16F, k, n, k);
    if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatrixLayoutCreate(&lc, HIP_R_32F, m, n, m);
  }
  ~LtDesc() {
    if (lc) hipblasLtMatrixLayoutDestroy(lc);
    if (lb) hipblasLtMatrixLayoutDestroy(lb);
    if (la) hipblasLtMatrixLayoutDestroy(la);
    if (md) hipblasLtMatmulDescDestroy(md);
  }
};

// C = A^T B (LtDesc) on stream s.  The algorithm of a shape is picked on its
// first call: the heuristic's first kLtCandidates algorithms are each run
// once, then timed over three calls on s (the host waits for s once per
// candidate), and the fastest is kept for every later call of that shape in
// this process, so repeated calls of a shape give identical results.  Another
// process may keep another algorithm: its sums differ in rounding only (fp32
// accumulation either way).  Beyond kLtMaxShapes shapes the heuristic's
// first algorithm is used untimed.
int lt_gemm(DevCtx *c, int m, int n, int k, const _Float16 *A, const _Float16 *B, float *C,
            hipStream_t s) {
  LtDesc d(m, n, k);
  if (d.st != HIPBLAS_STATUS_SUCCESS)
    return set_err(MIA_ERR_HIP, "hipBLASLt descriptors (%d x %d x %d): status %d", m, n, k, (int)d.st);
  const float one = 1.0f, zero = 0.0f;
  auto run = [&](const hipblasLtMatmulAlgo_t &algo) {
    return hipblasLtMatmul(c->lt, d.md, &one, A, d.la, B, d.lb, &zero, C, d.lc, C, d.lc, &algo,
                           c->lt_ws, kLtWorkspace, s);
  };
  for (const LtPick &p : c->lt_picks) {
    if (p.m != m || p.n != n || p.k != k) continue;
    const hipblasStatus_t st = run(p.algo);
    if (st != HIPBLAS_STATUS_SUCCESS) return set_err(MIA_ERR_HIP, "hipblasLtMatmul: status %d", (int)st);
    return MIA_OK;
  }
  hipblasLtMatmulPreference_t pref = nullptr;
  hipblasStatus_t st = hipblasLtMatmulPreferenceCreate(&pref);
  const uint64_t ws = kLtWorkspace;
  if (st == HIPBLAS_STATUS_SUCCESS)
    st = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                               sizeof(ws));
  hipblasLtMatmulHeuristicResult_t res[kLtCandidates];
  int got = 0;
  if (st == HIPBLAS_STATUS_SUCCESS)
    st = hipblasLtMatmulAlgoGetHeuristic(c->lt, d.md, d.la, d.lb, d.lc, d.lc, pref, kLtCandidates, res,
                                         &got);
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  if (st != HIPBLAS_STATUS_SUCCESS || got < 1)
    return set_err(MIA_ERR_HIP, "hipBLASLt: no algorithm for %d x %d x %d (status %d)", m, n, k, (int)st);
  int best = -1;
  const bool remember = c->lt_picks.size() < kLtMaxShapes;
  if (remember && got > 1) {
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t he = hipEventCreate(&e0);
    if (he == hipSuccess) he = hipEventCreate(&e1);
    float best_ms = 0.0f;
    for (int i = 0; he == hipSuccess && i < got; ++i) {
      if (res[i].state != HIPBLAS_STATUS_SUCCESS || res[i].workspaceSize > kLtWorkspace) continue;
      if (run(res[i].algo) != HIPBLAS_STATUS_SUCCESS) continue;
      he = hipEventRecord(e0, s);
      bool ok = true;
      for (int r = 0; r < 3 && ok; ++r) ok = run(res[i].algo) == HIPBLAS_STATUS_SUCCESS;
      if (he == hipSuccess) he = hipEventRecord(e1, s);
      if (he == hipSuccess) he = hipEventSynchronize(e1);
      float ms = 0.0f;
      if (he == hipSuccess) he = hipEventElapsedTime(&ms, e0, e1);
      if (he == hipSuccess && ok && (best < 0 || ms < best_ms)) {
        best = i;
        best_ms = ms;
      }
    }
    if (e1) (void)hipEventDestroy(e1);
    if (e0) (void)hipEventDestroy(e0);
    if (he != hipSuccess) return set_err(MIA_ERR_HIP, "timing the GEMM algorithms: %s", hipGetErrorString(he));
  }
  for (int i = 0; best < 0 && i < got; ++i)
    if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize <= kLtWorkspace) best = i;
  if (best < 0) return set_err(MIA_ERR_HIP, "hipBLASLt: no usable algorithm for %d x %d x %d", m, n, k);
  if (remember) c->lt_picks.push_back(LtPick{m, n, k, res[best].algo});
  st = run(res[best].algo);
  if (st != HIPBLAS_STATUS_SUCCESS) return set_err(MIA_ERR_HIP, "hipblasLtMatmul: status %d", (int)st);
  return MIA_OK;
}

int check_shape(int n_heads, int n_kv_heads, int hd, int max_seq) {
  if (n_heads <= 0 || n_kv_heads <= 0 || hd <= 0 || max_seq <= 0)
    return set_err(MIA_ERR_INVALID, "sizes must be positive (n_heads=%d n_kv_heads=%d hd=%d max_seq=%d)",
                   n_heads, n_kv_heads, hd, max_seq);
  if (n_heads % n_kv_heads)
    return set_err(MIA_ERR_INVALID, "n_heads %d not a multiple of n_kv_heads %d", n_heads, n_kv_heads);
  if (hd != kHD) return set_err(MIA_ERR_UNSUPPORTED, "head_dim %d unsupported (kernels need 128)", hd);
  if (n_heads / n_kv_heads != kG)
    return set_err(MIA_ERR_UNSUPPORTED, "GQA ratio %d unsupported (kernels need 4)", n_heads / n_kv_heads);
  if (max_seq > kMaxSeq) return set_err(MIA_ERR_UNSUPPORTED, "max_seq %d above %d", max_seq, kMaxSeq);
  if (n_kv_heads > 64) return set_err(MIA_ERR_UNSUPPORTED, "n_kv_heads %d above 64", n_kv_heads);
  return MIA_OK;
}

// The attention kernels move fp32 rows 16 bytes at a time.
int check_align16(const void *a, const void *b, const void *c, const void *d) {
  const uintptr_t bits = (uintptr_t)a | (uintptr_t)b | (uintptr_t)c | (uintptr_t)d;
  if (bits & 15) return set_err(MIA_ERR_INVALID, "Q/K/V/out device pointers must be 16-byte aligned");
  return MIA_OK;
}

int check_pos(int pos, int S) {
  if (pos < 0 || S < 1) return set_err(MIA_ERR_INVALID, "bad position %d / token count %d", pos, S);
  if ((long)pos + S >= (long)INT_MAX) return set_err(MIA_ERR_INVALID, "position %d + %d overflows", pos, S);
  return MIA_OK;
}

float qscale_log2() { return (1.0f / sqrtf((float)kHD)) * 1.4426950408889634f; }

// When timing is on, hands out the next event pair of this kind (created on
// demand); the launch stamps them at the main kernel's start and end.
int prof_pair(DevCtx *c, int kind, hipEvent_t *ev0, hipEvent_t *ev1) {
  *ev0 = *ev1 = nullptr;
  if (!c->prof_on) return MIA_OK;
  std::vector<hipEvent_t> &ev = c->prof_ev[kind];
  size_t idx = 2 * c->prof_n[kind];
  while (ev.size() < idx + 2) {
    hipEvent_t e;
    HIP_TRY(hipEventCreate(&e));
    ev.push_back(e);
  }
  *ev0 = ev[idx];
  *ev1 = ev[idx + 1];
  c->prof_n[kind]++;
  return MIA_OK;
}

// new_k / new_v (fused only, may be null): where the new token's fp16 rows go
// instead of its ring slot.  fixed (may be null): partials go there, at most
// fixed_bytes, instead of into the on-demand split area; the chunk count is
// capped to fit, and nothing is allocated (no timing events either).
int decode_impl(const float *q, const float *k, const float *v, const float *theta_inv,
                uint16_t *k_layer, uint16_t *v_layer, float *out, int n_heads, int n_kv, int max_seq,
                int pos, bool fused, void *stream, uint16_t *new_k = nullptr,
                uint16_t *new_v = nullptr, void *fixed = nullptr, size_t fixed_bytes = 0) {
  DevCtx *c;
  if (fixed != nullptr) {
    // no mia_init from here: it creates the library's stream
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices || !g_ctx[dev].ready)
      return set_err(MIA_ERR_NO_DEVICE, "device %d not initialised: call mia_init first", dev);
    c = &g_ctx[dev];
  } else if (int rc = current_ctx(&c)) {
    return rc;
  }
  const int L = pos + 1 < max_seq ? pos + 1 : max_seq;
  const long start = ((long)pos + 1 - L) % max_seq;
  mia::DecodeParams p{};
  p.q = q;
  p.knew = k;
  p.vnew = v;
  p.theta_inv = theta_inv;
  p.kc = reinterpret_cast<_Float16 *>(k_layer);
  p.vc = reinterpret_cast<_Float16 *>(v_layer);
  p.out = out;
  p.new_k = reinterpret_cast<_Float16 *>(new_k);
  p.new_v = reinterpret_cast<_Float16 *>(new_v);
  p.max_seq = max_seq;
  p.pos = pos;
  p.L = L;
  p.start = (int)start;
  p.new_slot = pos % max_seq;
  p.n_kv = n_kv;
  p.nchunk = mia::decode_pick_nchunk(L, n_kv, c->num_cus);
  if (fixed != nullptr) {
    const size_t per_chunk = mia::decode_scratch_bytes(n_kv, kG, 1);
    const size_t cap = fixed_bytes / per_chunk;
    if (cap < 2) p.nchunk = 1;  // a single chunk writes out directly
    else if ((size_t)p.nchunk > cap) p.nchunk = (int)cap;
  }
  p.qscale = qscale_log2();
  if (p.nchunk > 1) {
    if (fixed != nullptr) {
      p.part_o = reinterpret_cast<float *>(fixed);
    } else {
      if (int rc = ensure_scratch(c, mia::decode_scratch_bytes(n_kv, kG, p.nchunk))) return rc;
      p.part_o = reinterpret_cast<float *>(c->split);
    }
    p.part_ml = p.part_o + (size_t)n_kv * p.nchunk * kG * kHD;
  }
  hipStream_t s = pick_stream(c, stream);
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  if (fixed == nullptr) {
    if (int rc = prof_pair(c, 0, &ev0, &ev1)) return rc;
  }
  HIP_TRY(mia::launch_decode(p, kG, fused ? mia::kDecodeFused : mia::kDecodePlain, s, ev0, ev1));
  HIP_TRY(mia::launch_decode_merge(p, s));
  return MIA_OK;
}

// S tokens at their own positions (device int32 [S]) over the ring as it
// stands, through the decode kernel batched over tokens; theta_inv set: Q is
// raw and rotated in-kernel.  Every token takes the same chunk count, planned
// for the longest possible window (max_seq).
int positions_impl(DevCtx *c, const float *Q, const float *theta_inv, const int *positions,
                   const uint16_t *k_layer, const uint16_t *v_layer, float *out, int n_kv,
                   int max_seq, int S, hipStream_t s) {
  mia::DecodeParams p{};
  p.q = Q;
  p.theta_inv = theta_inv;
  p.kc = reinterpret_cast<_Float16 *>(const_cast<uint16_t *>(k_layer));
  p.vc = reinterpret_cast<_Float16 *>(const_cast<uint16_t *>(v_layer));
  p.out = out;
  p.max_seq = max_seq;
  p.n_kv = n_kv;
  p.positions = positions;
  p.n_tok = S;
  const int hgroups = (n_kv + 7) / 8;
  const int target = (c->num_cus + S * hgroups - 1) / (S * hgroups);
  p.nchunk = mia::decode_pick_nchunk(max_seq, n_kv, target * hgroups);
  p.qscale = qscale_log2();
  if (p.nchunk > 1) {
    if (int rc = ensure_scratch(c, mia::decode_scratch_bytes(n_kv, kG, p.nchunk, S))) return rc;
    p.part_o = reinterpret_cast<float *>(c->split);
    p.part_ml = p.part_o + (size_t)S * n_kv * p.nchunk * kG * kHD;
  }
  hipEvent_t ev0, ev1;
  if (int rc = prof_pair(c, 0, &ev0, &ev1)) return rc;
  HIP_TRY(mia::launch_decode(p, kG, mia::kDecodePositions, s, ev0, ev1));
  HIP_TRY(mia::launch_decode_merge(p, s));
  return MIA_OK;
}

int check_positions(const int *positions, int S) {
  if (!positions) return set_err(MIA_ERR_INVALID, "positions is NULL");
  if ((uintptr_t)positions & 3) return set_err(MIA_ERR_INVALID, "positions must be 4-byte aligned");
  if (S < 1 || S > 65535) return set_err(MIA_ERR_INVALID, "token count %d outside 1..65535", S);
  return MIA_OK;
}

// With commit, the staged drafts kst/vst are copied into the ring after the
// attention: by the split merge kernel when there is one, else by a copy
// kernel.
int flash_impl(DevCtx *c, const float *Q, const float *rope_cs, const uint16_t *kst,
               const uint16_t *vst, const uint16_t *k_layer, const uint16_t *v_layer, float *out,
               int n_kv, int max_seq, int start_pos, int S, hipStream_t s, bool commit = false) {
  mia::FlashParams p{};
  int rt = 0;
  mia::flash_plan(S, n_kv, kG, start_pos, max_seq, c->num_cus, &p.n_rtiles, &p.nsplit,
                  &p.split_keys, &rt);
  p.Q = Q;
  p.rope_cs = rope_cs;
  p.kc = reinterpret_cast<const _Float16 *>(k_layer);
  p.vc = reinterpret_cast<const _Float16 *>(v_layer);
  p.kstage = reinterpret_cast<const _Float16 *>(kst);
  p.vstage = reinterpret_cast<const _Float16 *>(vst);
  p.out = out;
  p.S = S;
  p.n_kv = n_kv;
  p.max_seq = max_seq;
  p.start_pos = start_pos;
  p.qscale = qscale_log2();
  if (p.nsplit > 1) {
    size_t ntile = (size_t)n_kv * p.n_rtiles;
    if (int rc = ensure_scratch(c, mia::flash_scratch_bytes(n_kv, p.n_rtiles, p.nsplit, rt)))
      return rc;
    p.part_o = reinterpret_cast<float *>(c->split);
    p.part_ml = p.part_o + ntile * p.nsplit * rt * kHD;
  }
  hipEvent_t ev0, ev1;
  if (int rc = prof_pair(c, 1, &ev0, &ev1)) return rc;
  if (commit && p.nsplit > 1) {
    p.commit_k = reinterpret_cast<_Float16 *>(const_cast<uint16_t *>(k_layer));
    p.commit_v = reinterpret_cast<_Float16 *>(const_cast<uint16_t *>(v_layer));
  }
  HIP_TRY(mia::launch_flash(p, kG, s, ev0, ev1));
  HIP_TRY(mia::launch_flash_merge(p, s));
  if (commit && p.nsplit == 1)
    HIP_TRY(mia::launch_commit(const_cast<_Float16 *>(p.kc), const_cast<_Float16 *>(p.vc),
                               p.kstage, p.vstage, S, start_pos, max_seq, n_kv * kHD, s));
  return MIA_OK;
}

// Q4_0 matvec over up to three stacked matrices; exactly one of x_q8 (Q8_0
// blocks) and xf (fp32, quantised in-kernel) is set.
int q4_impl(const void *Wq, const void *Wk, const void *Wv, const void *x_q8, const float *xf,
            float *yq, float *yk, float *yv, int dim, int kv_dim, int in_dim, void *stream) {
  if (!Wq || !(x_q8 || xf) || !yq || (kv_dim && (!Wk || !Wv || !yk || !yv)))
    return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (dim <= 0 || kv_dim < 0 || in_dim <= 0 || in_dim % 32)
    return set_err(MIA_ERR_INVALID, "bad sizes (dim=%d kv_dim=%d in_dim=%d)", dim, kv_dim, in_dim);
  if (in_dim % 64)
    return set_err(MIA_ERR_UNSUPPORTED, "in_dim %d: the kernel needs an even number of blocks per row",
                   in_dim);
  if (xf && in_dim > mia::kQ4MaxF32InDim)
    return set_err(MIA_ERR_UNSUPPORTED, "in_dim %d above %d for fp32 input (quantize first)", in_dim,
                   mia::kQ4MaxF32InDim);
  if ((long)dim + 2L * kv_dim > (long)INT_MAX) return set_err(MIA_ERR_INVALID, "too many rows");
  const uintptr_t bits = (uintptr_t)Wq | (uintptr_t)Wk | (uintptr_t)Wv | (uintptr_t)x_q8 |
                         (uintptr_t)yq | (uintptr_t)yk | (uintptr_t)yv;
  if (bits & 3) return set_err(MIA_ERR_INVALID, "weights, x_q8 and y must be 4-byte aligned");
  if ((uintptr_t)xf & 15) return set_err(MIA_ERR_INVALID, "x must be 16-byte aligned");
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  mia::Q4MatvecParams p{};
  p.w0 = reinterpret_cast<const uint8_t *>(Wq);
  p.w1 = reinterpret_cast<const uint8_t *>(Wk);
  p.w2 = reinterpret_cast<const uint8_t *>(Wv);
  p.y0 = yq;
  p.y1 = yk;
  p.y2 = yv;
  p.x = reinterpret_cast<const uint8_t *>(x_q8);
  p.xf = xf;
  p.rows0 = dim;
  p.rows01 = dim + kv_dim;
  p.total_rows = dim + 2 * kv_dim;
  p.bpr = in_dim / 32;
  hipEvent_t ev0, ev1;
  if (int rc = prof_pair(c, 2, &ev0, &ev1)) return rc;
  HIP_TRY(mia::launch_q4_matvec(p, pick_stream(c, stream), ev0, ev1));
  return MIA_OK;
}

}  // namespace

// Q4_0 GEMM over up to three stacked matrices (see GemmParams).
int gemm_impl(DevCtx *c, const void *W0, const void *W1, const void *W2, int rows0, int rows1,
              int rows2, const float *X, int K, int S, float *y0, float *y1, float *y2, int mode,
              hipStream_t s, bool reuse_split = false, const _Float16 *planes = nullptr,
              _Float16 *out_planes = nullptr, bool packed = false) {
  // X [S][K] as fp16 hi + lo planes in split_work; reuse_split: the planes of
  // the input are already there (written by the call before on this stream,
  // or by the RMSNorm that produced them), and X is not read.
  // planes: the input's planes given by the caller ([S][K] hi, then lo).
  // out_planes (kGemmSiluMul): the result as planes there instead of in y0.
  const size_t n = (size_t)S * K;
  const bool have = reuse_split || planes != nullptr;
  if (!have) {
    if (int rc = ensure_split_work(c, 2 * n * sizeof(_Float16))) return rc;
  }
  const _Float16 *const ahi =
      planes != nullptr ? planes : reinterpret_cast<const _Float16 *>(c->split_work);
  const _Float16 *const alo = ahi + n;
  if (!have)
    HIP_TRY(mia::launch_split_hilo(X, (long)n, const_cast<_Float16 *>(ahi),
                                   const_cast<_Float16 *>(alo), c->num_cus, s));
  mia::GemmParams p{};
  p.ahi = ahi;
  p.alo = alo;
  if (out_planes != nullptr) {
    p.ohi = out_planes;
    p.olo = out_planes + (size_t)S * (rows0 + rows1 + rows2);
  }
  p.w0 = reinterpret_cast<const uint8_t *>(W0);
  p.w1 = reinterpret_cast<const uint8_t *>(W1);
  p.w2 = reinterpret_cast<const uint8_t *>(W2);
  p.rows0 = rows0;
  p.rows01 = rows0 + rows1;
  p.N = rows0 + rows1 + rows2;
  p.K = K;
  p.S = S;
  p.y0 = y0;
  p.y1 = y1;
  p.y2 = y2;
  p.packed = packed ? 1 : 0;
  p.ksplit = mia::gemm_pick_ksplit(p.N, K, S, c->num_cus);
  if (p.ksplit > 1) {
    if (int rc = ensure_gemm_work(c, (size_t)p.ksplit * S * p.N * sizeof(float))) return rc;
    p.part = reinterpret_cast<float *>(c->gemm_work);
  }
  hipEvent_t ev0, ev1;
  if (int rc = prof_pair(c, 3, &ev0, &ev1)) return rc;
  HIP_TRY(mia::launch_q4_gemm(p, mode, c->num_cus, s, ev0, ev1));
  return MIA_OK;
}

int check_gemm_dims(int out_dim, int in_dim, int S) {
  if (out_dim <= 0 || in_dim <= 0 || S <= 0 || in_dim % 32)
    return set_err(MIA_ERR_INVALID, "bad sizes (out_dim=%d in_dim=%d S=%d)", out_dim, in_dim, S);
  if (in_dim % 64)
    return set_err(MIA_ERR_UNSUPPORTED, "in_dim %d: the GEMM needs a multiple of 64", in_dim);
  if ((long)S * in_dim > INT_MAX || (long)S * out_dim > INT_MAX)
    return set_err(MIA_ERR_UNSUPPORTED, "S x dim above 2^31");
  return MIA_OK;
}

// Error reporting for the library's C sources (not exported).
extern "C" __attribute__((visibility("hidden"))) int mia_internal_set_error(int code,
                                                                            const char *msg) {
  return set_err(code, "%s", msg);
}

// Pinned host memory and stream-ordered copies for the drop-in's staging
// (mia_dropin.c): one transfer each way per call, on the library stream the
// kernels of a NULL-stream call run on.
extern "C" __attribute__((visibility("hidden"))) int mia_internal_host_alloc(void **p,
                                                                             size_t bytes) {
  if (!p || bytes == 0) return set_err(MIA_ERR_INVALID, "host_alloc: NULL pointer or 0 bytes");
  HIP_TRY(hipHostMalloc(p, bytes, hipHostMallocDefault));
  return MIA_OK;
}

extern "C" __attribute__((visibility("hidden"))) int mia_internal_host_free(void *p) {
  if (p) HIP_TRY(hipHostFree(p));
  return MIA_OK;
}

extern "C" __attribute__((visibility("hidden"))) int mia_internal_copy_async(void *dst,
                                                                             const void *src,
                                                                             size_t bytes,
                                                                             int to_device) {
  if (bytes == 0) return MIA_OK;
  if (!dst || !src) return set_err(MIA_ERR_INVALID, "NULL pointer");
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  HIP_TRY(hipMemcpyAsync(dst, src, bytes, to_device ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost,
                         c->stream));
  return MIA_OK;
}

extern "C" {

int mia_version(void) { return 100; }

const char *mia_last_error(void) { return g_err; }

int mia_device_count(int *count) {
  if (!count) return set_err(MIA_ERR_INVALID, "count is NULL");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) {
    *count = 0;
    return set_err(MIA_ERR_NO_DEVICE, "hipGetDeviceCount: %s", hipGetErrorString(e));
  }
  *count = n;
  return MIA_OK;
}

int mia_init(int device) {
  std::lock_guard<std::mutex> lock(g_mu);
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= 0)
    return set_err(MIA_ERR_NO_DEVICE, "no HIP device: %s", hipGetErrorString(e));
  if (device < 0 || device >= n || device >= kMaxDevices)
    return set_err(MIA_ERR_INVALID, "device %d out of range (%d devices)", device, n);
  HIP_TRY(hipSetDevice(device));
  DevCtx &c = g_ctx[device];
  if (c.ready) return MIA_OK;
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return set_err(MIA_ERR_UNSUPPORTED, "device %d is %s; libmiattn is built for gfx950", device,
                   prop.gcnArchName);
  c.num_cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
  HIP_TRY(mia::prepare_flash());
  HIP_TRY(mia::prepare_gemm());
  HIP_TRY(hipGetSymbolAddress(&c.noalloc, HIP_SYMBOL(scratch)));
  HIP_TRY(hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking));
  c.ready = true;
  return MIA_OK;
}

int mia_profile_begin(void) {
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  for (size_t &n : c->prof_n) n = 0;
  c->prof_on = true;
  return MIA_OK;
}

int mia_profile_end(int kind, int *count, double *total_ms) {
  if (kind < 0 || kind > 5 || !count || !total_ms) return set_err(MIA_ERR_INVALID, "bad profile query");
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  c->prof_on = false;
  HIP_TRY(hipDeviceSynchronize());
  double total = 0.0;
  for (size_t i = 0; i < c->prof_n[kind]; ++i) {
    float ms = 0.f;
    HIP_TRY(hipEventElapsedTime(&ms, c->prof_ev[kind][2 * i], c->prof_ev[kind][2 * i + 1]));
    total += ms;
  }
  *count = (int)c->prof_n[kind];
  *total_ms = total;
  return MIA_OK;
}

int mia_malloc(void **dptr, size_t bytes) {
  if (!dptr) return set_err(MIA_ERR_INVALID, "dptr is NULL");
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  HIP_TRY(hipMalloc(dptr, bytes ? bytes : 1));
  return MIA_OK;
}

int mia_free(void *dptr) {
  if (dptr) HIP_TRY(hipFree(dptr));
  return MIA_OK;
}

int mia_memcpy_h2d(void *dst, const void *src, size_t bytes) {
  if (bytes == 0) return MIA_OK;
  if (!dst || !src) return set_err(MIA_ERR_INVALID, "NULL pointer");
  HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return MIA_OK;
}

int mia_memcpy_d2h(void *dst, const void *src, size_t bytes) {
  if (bytes == 0) return MIA_OK;
  if (!dst || !src) return set_err(MIA_ERR_INVALID, "NULL pointer");
  HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return MIA_OK;
}

int mia_memcpy_d2d(void *dst, const void *src, size_t bytes) {
  if (bytes == 0) return MIA_OK;
  if (!dst || !src) return set_err(MIA_ERR_INVALID, "NULL pointer");
  HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
  return MIA_OK;
}

int mia_memset(void *dst, int value, size_t bytes) {
  if (bytes == 0) return MIA_OK;
  if (!dst) return set_err(MIA_ERR_INVALID, "NULL pointer");
  HIP_TRY(hipMemset(dst, value, bytes));
  return MIA_OK;
}

int mia_stream_create(void **stream) {
  if (!stream) return set_err(MIA_ERR_INVALID, "stream is NULL");
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  hipStream_t s;
  HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *stream = s;
  return MIA_OK;
}

int mia_stream_destroy(void *stream) {
  if (stream) HIP_TRY(hipStreamDestroy(reinterpret_cast<hipStream_t>(stream)));
  return MIA_OK;
}

int mia_stream_sync(void *stream) {
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  HIP_TRY(hipStreamSynchronize(pick_stream(c, stream)));
  return MIA_OK;
}

int mia_device_sync(void) {
  HIP_TRY(hipDeviceSynchronize());
  return MIA_OK;
}

int mia_event_create(void **event) {
  if (!event) return set_err(MIA_ERR_INVALID, "event is NULL");
  hipEvent_t e;
  HIP_TRY(hipEventCreate(&e));
  *event = e;
  return MIA_OK;
}

int mia_event_destroy(void *event) {
  if (event) HIP_TRY(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)));
  return MIA_OK;
}

int mia_event_record(void *event, void *stream) {
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  HIP_TRY(hipEventRecord(reinterpret_cast<hipEvent_t>(event), pick_stream(c, stream)));
  return MIA_OK;
}

int mia_event_elapsed_ms(float *ms, void *start, void *stop) {
  if (!ms) return set_err(MIA_ERR_INVALID, "ms is NULL");
  HIP_TRY(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                              reinterpret_cast<hipEvent_t>(stop)));
  return MIA_OK;
}

int mia_fill_normal_f16(uint16_t *dst, size_t n, uint64_t seed, void *stream) {
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  if (!dst && n) return set_err(MIA_ERR_INVALID, "dst is NULL");
  HIP_TRY(mia::launch_fill_normal(reinterpret_cast<_Float16 *>(dst), n, seed, pick_stream(c, stream)));
  return MIA_OK;
}

int mia_peak_read_stream(const void *buf, size_t bytes, void *stream) {
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  if (!buf || bytes == 0 || bytes % 16 != 0)
    return set_err(MIA_ERR_INVALID, "peak_read_stream: need a buffer of a positive multiple of 16 bytes");
  HIP_TRY(mia::launch_peak_read_stream(buf, bytes, c->num_cus, pick_stream(c, stream)));
  return MIA_OK;
}

int mia_peak_read_ring(const uint16_t *k_layer, const uint16_t *v_layer, int n_kv_heads,
                       int max_seq, int L, int start, void *stream) {
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  if (!k_layer || !v_layer) return set_err(MIA_ERR_INVALID, "peak_read_ring: NULL ring");
  if (n_kv_heads < 1 || max_seq < 1 || L < 1 || L > max_seq || start < 0 || start >= max_seq)
    return set_err(MIA_ERR_INVALID, "peak_read_ring: need 1 <= L <= max_seq, 0 <= start < max_seq");
  const int nchunk = mia::decode_pick_nchunk(L, n_kv_heads, c->num_cus);
  HIP_TRY(mia::launch_peak_read_ring(reinterpret_cast<const _Float16 *>(k_layer),
                                     reinterpret_cast<const _Float16 *>(v_layer), n_kv_heads,
                                     max_seq, L, start, nchunk, pick_stream(c, stream)));
  return MIA_OK;
}

int mia_peak_mfma_f16(int iters, double *flop, void *stream) {
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  if (iters < 1 || !flop) return set_err(MIA_ERR_INVALID, "peak_mfma_f16: iters >= 1 and flop");
  HIP_TRY(mia::launch_peak_mfma_f16(iters, c->num_cus, flop, pick_stream(c, stream)));
  return MIA_OK;
}

int mia_peak_empty(int workgroups, int threads, void *stream) {
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  if (workgroups < 1 || threads < 1 || threads > 1024)
    return set_err(MIA_ERR_INVALID, "peak_empty: need workgroups >= 1 and 1 <= threads <= 1024");
  hipEvent_t ev0, ev1;
  if (int rc = prof_pair(c, 4, &ev0, &ev1)) return rc;
  HIP_TRY(mia::launch_peak_empty(workgroups, threads, pick_stream(c, stream), ev0, ev1));
  return MIA_OK;
}

int mia_scale_rows_f16(uint16_t *base, long n_rows, int row_elems, int every, int offset,
                       float factor, void *stream) {
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  if (!base || n_rows < 0 || row_elems <= 0 || every <= 0 || offset < 0)
    return set_err(MIA_ERR_INVALID, "bad scale_rows arguments");
  HIP_TRY(mia::launch_scale_rows(reinterpret_cast<_Float16 *>(base), n_rows, row_elems, every,
                                 offset, factor, pick_stream(c, stream)));
  return MIA_OK;
}

int mia_rope_f32(float *q, float *k, int S, int start_pos, const float *theta_inv, int n_heads,
                 int n_kv_heads, int head_dim, void *stream) {
  if (head_dim != kHD) return set_err(MIA_ERR_UNSUPPORTED, "head_dim %d unsupported", head_dim);
  if (!theta_inv) return set_err(MIA_ERR_INVALID, "theta_inv is NULL");
  if ((q && n_heads <= 0) || (k && n_kv_heads <= 0)) return set_err(MIA_ERR_INVALID, "bad head counts");
  if (int rc = check_pos(start_pos, S)) return rc;
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  HIP_TRY(mia::launch_rope(q, k, S, start_pos, theta_inv, q ? n_heads : 0, k ? n_kv_heads : 0,
                           pick_stream(c, stream)));
  return MIA_OK;
}

int mia_kv_write_f32(uint16_t *k_layer, uint16_t *v_layer, const float *K, const float *V, int S,
                     int start_pos, int max_seq, int kv_dim, void *stream) {
  if (!k_layer || !v_layer || !K || !V) return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (kv_dim <= 0 || max_seq <= 0 || max_seq > kMaxSeq) return set_err(MIA_ERR_INVALID, "bad kv_dim/max_seq");
  if (int rc = check_pos(start_pos, S)) return rc;
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  HIP_TRY(mia::launch_kv_write(reinterpret_cast<_Float16 *>(k_layer),
                               reinterpret_cast<_Float16 *>(v_layer), K, V, S, start_pos, max_seq,
                               kv_dim, pick_stream(c, stream)));
  return MIA_OK;
}

int mia_gqa_attention(const float *q, float *out, const uint16_t *k_layer, const uint16_t *v_layer,
                      int n_heads, int heads_per_kv, int hd, int max_seq, int pos, void *stream) {
  if (!q || !out || !k_layer || !v_layer) return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (heads_per_kv <= 0) return set_err(MIA_ERR_INVALID, "heads_per_kv %d", heads_per_kv);
  const int n_kv = n_heads / heads_per_kv;
  if (n_kv * heads_per_kv != n_heads) return set_err(MIA_ERR_INVALID, "n_heads/heads_per_kv mismatch");
  if (int rc = check_shape(n_heads, n_kv, hd, max_seq)) return rc;
  if (int rc = check_pos(pos, 1)) return rc;
  return decode_impl(q, nullptr, nullptr, nullptr, const_cast<uint16_t *>(k_layer),
                     const_cast<uint16_t *>(v_layer), out, n_heads, n_kv, max_seq, pos, false, stream);
}

int mia_decode_step(const float *q, const float *k, const float *v, const float *theta_inv,
                    uint16_t *k_layer, uint16_t *v_layer, float *out, int n_heads, int n_kv_heads,
                    int hd, int max_seq, int pos, void *stream) {
  if (!q || !k || !v || !theta_inv || !out || !k_layer || !v_layer)
    return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (int rc = check_shape(n_heads, n_kv_heads, hd, max_seq)) return rc;
  if (int rc = check_pos(pos, 1)) return rc;
  return decode_impl(q, k, v, theta_inv, k_layer, v_layer, out, n_heads, n_kv_heads, max_seq, pos,
                     true, stream);
}

int mia_decode_step_noalloc(const float *q, const float *k, const float *v,
                            const float *theta_inv, uint16_t *k_layer, uint16_t *v_layer,
                            float *out, int n_heads, int n_kv_heads, int hd, int max_seq, int pos,
                            void *stream) {
  if (!q || !k || !v || !theta_inv || !out || !k_layer || !v_layer)
    return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (int rc = check_shape(n_heads, n_kv_heads, hd, max_seq)) return rc;
  if (int rc = check_pos(pos, 1)) return rc;
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices || !g_ctx[dev].ready || g_ctx[dev].noalloc == nullptr)
    return set_err(MIA_ERR_NO_DEVICE, "device %d not initialised: call mia_init first", dev);
  return decode_impl(q, k, v, theta_inv, k_layer, v_layer, out, n_heads, n_kv_heads, max_seq, pos,
                     true, stream, nullptr, nullptr, g_ctx[dev].noalloc, kNoAllocScratchBytes);
}

int mia_attention_batch(const float *Q, float *out, const uint16_t *k_layer, const uint16_t *v_layer,
                        int n_heads, int n_kv_heads, int hd, int max_seq, int start_pos, int S,
                        void *stream) {
  if (!Q || !out || !k_layer || !v_layer) return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (int rc = check_align16(Q, out, k_layer, v_layer)) return rc;
  if (int rc = check_shape(n_heads, n_kv_heads, hd, max_seq)) return rc;
  if (int rc = check_pos(start_pos, S)) return rc;
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  return flash_impl(c, Q, nullptr, nullptr, nullptr, k_layer, v_layer, out, n_kv_heads, max_seq,
                    start_pos, S, pick_stream(c, stream));
}

int mia_attention_positions(const float *Q, float *out, const uint16_t *k_layer,
                            const uint16_t *v_layer, const int *positions, int n_heads,
                            int n_kv_heads, int hd, int max_seq, int S, void *stream) {
  if (!Q || !out || !k_layer || !v_layer) return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (int rc = check_positions(positions, S)) return rc;
  if (int rc = check_align16(Q, out, k_layer, v_layer)) return rc;
  if (int rc = check_shape(n_heads, n_kv_heads, hd, max_seq)) return rc;
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  return positions_impl(c, Q, nullptr, positions, k_layer, v_layer, out, n_kv_heads, max_seq, S,
                        pick_stream(c, stream));
}

int mia_attention_chunk(const float *Q, const float *K, const float *V, const int *positions,
                        const float *theta_inv, uint16_t *k_layer, uint16_t *v_layer, float *out,
                        int n_heads, int n_kv_heads, int hd, int max_seq, int S, void *stream) {
  if (!Q || !K || !V || !theta_inv || !out || !k_layer || !v_layer)
    return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (int rc = check_positions(positions, S)) return rc;
  if (int rc = check_align16(Q, K, V, out)) return rc;
  if (int rc = check_align16(k_layer, v_layer, nullptr, nullptr)) return rc;
  if (int rc = check_shape(n_heads, n_kv_heads, hd, max_seq)) return rc;
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  hipStream_t s = pick_stream(c, stream);
  // phase 1 (mistral_model.h:935-955), then phase 2 (:961-1044) with Q
  // rotated in the attention kernel.  Which token of a slot writes last: a
  // scan of the later tokens for short chunks (the reference's are 32,
  // mistral_model.h:902), one linear pass through a per-slot area beyond.
  int *owner = nullptr;
  if (S > kChunkScanMax) {
    if (int rc = ensure_owner(c, max_seq)) return rc;
    owner = c->owner;
  }
  HIP_TRY(mia::launch_rope_kv_positions(K, V, theta_inv, positions, S, n_kv_heads,
                                        reinterpret_cast<_Float16 *>(k_layer),
                                        reinterpret_cast<_Float16 *>(v_layer), max_seq, owner,
                                        s));
  return positions_impl(c, Q, theta_inv, positions, k_layer, v_layer, out, n_kv_heads, max_seq, S,
                        s);
}

int mia_attention_step(const float *Q, const float *K, const float *V, const float *theta_inv,
                       uint16_t *k_layer, uint16_t *v_layer, float *out, int n_heads,
                       int n_kv_heads, int hd, int max_seq, int start_pos, int S, void *stream) {
  if (!Q || !K || !V || !theta_inv || !out || !k_layer || !v_layer)
    return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (int rc = check_shape(n_heads, n_kv_heads, hd, max_seq)) return rc;
  if (int rc = check_pos(start_pos, S)) return rc;
  if (S > 1) {
    if (int rc = check_align16(Q, K, V, out)) return rc;
    if (int rc = check_align16(k_layer, v_layer, nullptr, nullptr)) return rc;
  }
  if (S == 1)
    return decode_impl(Q, K, V, theta_inv, k_layer, v_layer, out, n_heads, n_kv_heads, max_seq,
                       start_pos, true, stream);
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  hipStream_t s = pick_stream(c, stream);
  const int kv_dim = n_kv_heads * kHD;
  // Drafts may go straight into the ring when no slot they take still holds
  // a position some query of the batch attends (start_pos + S <= max_seq).
  // The K rotation also leaves the (cos, sin) table of the positions in the
  // work buffer, from which the attention kernel rotates Q.
  const bool direct = (long)start_pos + S <= (long)max_seq;
  const size_t cs_bytes = (size_t)S * kHD * sizeof(float);  // S x 64 (cos, sin)
  const size_t st_bytes = direct ? 0 : (size_t)S * kv_dim * sizeof(uint16_t);
  if (int rc = ensure_work(c, cs_bytes + 2 * st_bytes)) return rc;
  float *cs = reinterpret_cast<float *>(c->work);
  if (direct) {
    HIP_TRY(mia::launch_rope_to_ring(K, V, theta_inv, S, start_pos, n_kv_heads,
                                     reinterpret_cast<_Float16 *>(k_layer),
                                     reinterpret_cast<_Float16 *>(v_layer), max_seq, cs, s));
    return flash_impl(c, Q, cs, nullptr, nullptr, k_layer, v_layer, out, n_kv_heads, max_seq,
                      start_pos, S, s);
  }
  _Float16 *kst = reinterpret_cast<_Float16 *>(reinterpret_cast<char *>(c->work) + cs_bytes);
  _Float16 *vst = kst + (size_t)S * kv_dim;
  HIP_TRY(mia::launch_rope_to_f16(K, V, theta_inv, S, start_pos, n_kv_heads, kst, vst, cs, s));
  return flash_impl(c, Q, cs, reinterpret_cast<uint16_t *>(kst),
                    reinterpret_cast<uint16_t *>(vst), k_layer, v_layer, out, n_kv_heads, max_seq,
                    start_pos, S, s, true);
}

int mia_attention_step_staged(const float *Q, const float *K, const float *V,
                              const float *theta_inv, const uint16_t *k_layer,
                              const uint16_t *v_layer, uint16_t *k_stage, uint16_t *v_stage,
                              float *out, int n_heads, int n_kv_heads, int hd, int max_seq,
                              int start_pos, int S, void *stream) {
  if (!Q || !K || !V || !theta_inv || !out || !k_layer || !v_layer || !k_stage || !v_stage)
    return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (int rc = check_shape(n_heads, n_kv_heads, hd, max_seq)) return rc;
  if (int rc = check_pos(start_pos, S)) return rc;
  if (int rc = check_align16(Q, K, V, out)) return rc;
  if (int rc = check_align16(k_layer, v_layer, k_stage, v_stage)) return rc;
  if (S == 1)
    return decode_impl(Q, K, V, theta_inv, const_cast<uint16_t *>(k_layer),
                       const_cast<uint16_t *>(v_layer), out, n_heads, n_kv_heads, max_seq,
                       start_pos, true, stream, k_stage, v_stage);
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  hipStream_t s = pick_stream(c, stream);
  const size_t cs_bytes = (size_t)S * kHD * sizeof(float);  // S x 64 (cos, sin)
  if (int rc = ensure_work(c, cs_bytes)) return rc;
  float *cs = reinterpret_cast<float *>(c->work);
  HIP_TRY(mia::launch_rope_to_f16(K, V, theta_inv, S, start_pos, n_kv_heads,
                                  reinterpret_cast<_Float16 *>(k_stage),
                                  reinterpret_cast<_Float16 *>(v_stage), cs, s));
  return flash_impl(c, Q, cs, k_stage, v_stage, k_layer, v_layer, out, n_kv_heads, max_seq,
                    start_pos, S, s);
}

int mia_commit_staged(uint16_t *k_cache, uint16_t *v_cache, const uint16_t *k_stage,
                      const uint16_t *v_stage, int n_layers, int S_staged, int n_keep,
                      int start_pos, int max_seq, int kv_dim, void *stream) {
  if (!k_cache || !v_cache || !k_stage || !v_stage) return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (n_layers <= 0 || n_layers > 1024 || S_staged <= 0 || n_keep < 0 || n_keep > S_staged)
    return set_err(MIA_ERR_INVALID, "bad counts (n_layers=%d S_staged=%d n_keep=%d)", n_layers,
                   S_staged, n_keep);
  if (kv_dim <= 0 || kv_dim % 8 || max_seq <= 0 || max_seq > kMaxSeq)
    return set_err(MIA_ERR_INVALID, "bad kv_dim/max_seq");
  if (n_keep > max_seq) return set_err(MIA_ERR_INVALID, "n_keep %d above max_seq %d", n_keep, max_seq);
  if (int rc = check_pos(start_pos, S_staged)) return rc;
  if (int rc = check_align16(k_cache, v_cache, k_stage, v_stage)) return rc;
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  HIP_TRY(mia::launch_commit(reinterpret_cast<_Float16 *>(k_cache),
                             reinterpret_cast<_Float16 *>(v_cache),
                             reinterpret_cast<const _Float16 *>(k_stage),
                             reinterpret_cast<const _Float16 *>(v_stage), n_keep, start_pos,
                             max_seq, kv_dim, pick_stream(c, stream), n_layers,
                             (size_t)max_seq * kv_dim, (size_t)S_staged * kv_dim));
  return MIA_OK;
}

int mia_rmsnorm_f32(float *out, const float *in, const float *w, int dim, int S, float eps,
                    void *stream) {
  if (!out || !in || !w) return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (dim <= 0 || dim % 4 || S <= 0) return set_err(MIA_ERR_INVALID, "bad sizes (dim=%d S=%d)", dim, S);
  if (int rc = check_align16(out, in, w, nullptr)) return rc;
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  HIP_TRY(mia::launch_rmsnorm(out, in, w, dim, S, eps, pick_stream(c, stream)));
  return MIA_OK;
}

int mia_q4_0_gemm_f32(const void *W, const float *X, float *Y, int out_dim, int in_dim, int S,
                      void *stream) {
  if (!W || !X || !Y) return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (int rc = check_gemm_dims(out_dim, in_dim, S)) return rc;
  if ((uintptr_t)W & 3) return set_err(MIA_ERR_INVALID, "W must be 4-byte aligned");
  if (int rc = check_align16(X, Y, nullptr, nullptr)) return rc;
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  return gemm_impl(c, W, nullptr, nullptr, out_dim, 0, 0, X, in_dim, S, Y, nullptr, nullptr,
                   mia::kGemmStore, pick_stream(c, stream));
}

int mia_q4_0_pack_gemm(const void *W, void *Wp, int out_dim, int in_dim, void *stream) {
  if (!W || !Wp) return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (out_dim <= 0 || in_dim <= 0 || out_dim % 64 || in_dim % 64)
    return set_err(MIA_ERR_INVALID, "out_dim %d and in_dim %d must be positive multiples of 64",
                   out_dim, in_dim);
  if ((uintptr_t)W & 3) return set_err(MIA_ERR_INVALID, "W must be 4-byte aligned");
  if ((uintptr_t)Wp & 15) return set_err(MIA_ERR_INVALID, "Wp must be 16-byte aligned");
  const uintptr_t bytes = (uintptr_t)out_dim * (uintptr_t)(in_dim / 32) * 18;
  const uintptr_t a = (uintptr_t)W, b = (uintptr_t)Wp;
  if (a < b + bytes && b < a + bytes) return set_err(MIA_ERR_INVALID, "W and Wp overlap");
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  HIP_TRY(mia::launch_q4_pack(W, Wp, out_dim, in_dim, pick_stream(c, stream)));
  return MIA_OK;
}

int mia_q4_0_gemm_packed_f32(const void *Wp, const float *X, float *Y, int out_dim, int in_dim,
                             int S, void *stream) {
  if (!Wp || !X || !Y) return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (int rc = check_gemm_dims(out_dim, in_dim, S)) return rc;
  if (out_dim % 64) return set_err(MIA_ERR_INVALID, "out_dim %d must be a multiple of 64", out_dim);
  if ((uintptr_t)Wp & 15) return set_err(MIA_ERR_INVALID, "Wp must be 16-byte aligned");
  if (int rc = check_align16(X, Y, nullptr, nullptr)) return rc;
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  return gemm_impl(c, Wp, nullptr, nullptr, out_dim, 0, 0, X, in_dim, S, Y, nullptr, nullptr,
                   mia::kGemmStore, pick_stream(c, stream), false, nullptr, nullptr, true);
}

// (every row count, dim, kv_dim and hidden, is a multiple of 64 here, as the
// tile layout needs)
static int prefill_layer_impl(float *X, const mia_layer_weights *lw, const float *theta_inv,
                       uint16_t *k_layer, uint16_t *v_layer, int dim, int hidden, int n_heads,
                       int n_kv_heads, float eps, int max_seq, int start_pos, int S, void *stream,
                       bool packed) {
  if (!X || !lw || !theta_inv || !k_layer || !v_layer) return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (!lw->wq || !lw->wk || !lw->wv || !lw->wo || !lw->w1 || !lw->w2 || !lw->w3 || !lw->rms_att ||
      !lw->rms_ffn)
    return set_err(MIA_ERR_INVALID, "NULL weight pointer");
  if (n_heads <= 0 || dim != n_heads * kHD)
    return set_err(MIA_ERR_UNSUPPORTED, "dim %d must be n_heads x 128", dim);
  if (int rc = check_shape(n_heads, n_kv_heads, kHD, max_seq)) return rc;
  if (int rc = check_pos(start_pos, S)) return rc;
  if (int rc = check_gemm_dims(hidden, dim, S)) return rc;
  if (int rc = check_gemm_dims(dim, hidden, S)) return rc;
  const uintptr_t wb = (uintptr_t)lw->wq | (uintptr_t)lw->wk | (uintptr_t)lw->wv |
                       (uintptr_t)lw->wo | (uintptr_t)lw->w1 | (uintptr_t)lw->w2 |
                       (uintptr_t)lw->w3;
  if (wb & (packed ? 15 : 3))
    return set_err(MIA_ERR_INVALID, "weights must be %d-byte aligned", packed ? 16 : 4);
  if (int rc = check_align16(X, lw->rms_att, lw->rms_ffn, k_layer)) return rc;
  if (int rc = check_align16(v_layer, nullptr, nullptr, nullptr)) return rc;
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  hipStream_t s = pick_stream(c, stream);
  const int kv_dim = n_kv_heads * kHD;
  // Q [S][dim] | K, V [S][kv_dim] | A [S][dim] | G [S][hidden] | H planes
  // [2][S][hidden] fp16; the normalised rows (the QKV and W1 / W3 inputs) only
  // exist as the GEMM's hi + lo planes in split_work, written there by the
  // RMSNorm, and the SwiGLU output H (W2's input) only as the planes after G.
  auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
  const size_t bd = al((size_t)S * dim * 4), bk = al((size_t)S * kv_dim * 4),
               bh = al((size_t)S * hidden * 4);
  if (int rc = ensure_layer_work(c, 2 * bd + 2 * bk + 2 * bh)) return rc;
  if (int rc = ensure_split_work(c, (size_t)S * dim * 4)) return rc;  // [2][S][dim] fp16
  char *w = reinterpret_cast<char *>(c->layer_work);
  float *Q = reinterpret_cast<float *>(w);
  float *K = reinterpret_cast<float *>(w + bd);
  float *V = reinterpret_cast<float *>(w + bd + bk);
  float *A = reinterpret_cast<float *>(w + bd + 2 * bk);
  float *G = reinterpret_cast<float *>(w + 2 * bd + 2 * bk);
  _Float16 *const h_planes = reinterpret_cast<_Float16 *>(w + 2 * bd + 2 * bk + bh);
  _Float16 *const xn_hi = reinterpret_cast<_Float16 *>(c->split_work);
  _Float16 *const xn_lo = xn_hi + (size_t)S * dim;
  // mistral_ane_prefill.h:1092-1110
  HIP_TRY(mia::launch_rmsnorm_split(xn_hi, xn_lo, X, lw->rms_att, dim, S, eps, s));
  if (int rc = gemm_impl(c, lw->wq, lw->wk, lw->wv, dim, kv_dim, kv_dim, nullptr, dim, S, Q, K,
                         V, mia::kGemmStore, s, /*reuse_split=*/true, nullptr, nullptr, packed))
    return rc;
  // apply_rope_batch, kv_write_batch, attention_batch (:1097-1098): every
  // token's K/V go into the ring first and each query attends the ring as
  // it then stands; the (cos, sin) table of the positions lands in the work
  // buffer, from which the attention kernel rotates Q.
  if (int rc = ensure_work(c, (size_t)S * kHD * sizeof(float))) return rc;
  float *cs = reinterpret_cast<float *>(c->work);
  HIP_TRY(mia::launch_rope_to_ring(K, V, theta_inv, S, start_pos, n_kv_heads,
                                   reinterpret_cast<_Float16 *>(k_layer),
                                   reinterpret_cast<_Float16 *>(v_layer), max_seq, cs, s));
  if (int rc = flash_impl(c, Q, cs, nullptr, nullptr, k_layer, v_layer, A, n_kv_heads, max_seq,
                          start_pos, S, s))
    return rc;
  if (int rc = gemm_impl(c, lw->wo, nullptr, nullptr, dim, 0, 0, A, dim, S, X, nullptr, nullptr,
                         mia::kGemmAdd, s, false, nullptr, nullptr, packed))
    return rc;
  HIP_TRY(mia::launch_rmsnorm_split(xn_hi, xn_lo, X, lw->rms_ffn, dim, S, eps, s));
  if (int rc = gemm_impl(c, lw->w1, nullptr, nullptr, hidden, 0, 0, nullptr, dim, S, G, nullptr,
                         nullptr, mia::kGemmStore, s, /*reuse_split=*/true, nullptr, nullptr,
                         packed))
    return rc;
  if (int rc = gemm_impl(c, lw->w3, nullptr, nullptr, hidden, 0, 0, nullptr, dim, S, G, nullptr,
                         nullptr, mia::kGemmSiluMul, s, /*reuse_split=*/true, nullptr, h_planes,
                         packed))
    return rc;
  return gemm_impl(c, lw->w2, nullptr, nullptr, dim, 0, 0, nullptr, hidden, S, X, nullptr,
                   nullptr, mia::kGemmAdd, s, false, h_planes, nullptr, packed);
}

int mia_prefill_layer(float *X, const mia_layer_weights *lw, const float *theta_inv,
                      uint16_t *k_layer, uint16_t *v_layer, int dim, int hidden, int n_heads,
                      int n_kv_heads, float eps, int max_seq, int start_pos, int S,
                      void *stream) {
  return prefill_layer_impl(X, lw, theta_inv, k_layer, v_layer, dim, hidden, n_heads, n_kv_heads,
                            eps, max_seq, start_pos, S, stream, false);
}

int mia_prefill_layer_packed(float *X, const mia_layer_weights *lw, const float *theta_inv,
                             uint16_t *k_layer, uint16_t *v_layer, int dim, int hidden,
                             int n_heads, int n_kv_heads, float eps, int max_seq, int start_pos,
                             int S, void *stream) {
  return prefill_layer_impl(X, lw, theta_inv, k_layer, v_layer, dim, hidden, n_heads, n_kv_heads,
                            eps, max_seq, start_pos, S, stream, true);
}

// ---- weight types other than Q4_0 ------------------------------------------

static int check_typed(int type, int in_dim, const void *W) {
  if (mia::typed_row_bytes(type, in_dim) == 0)
    return set_err(MIA_ERR_UNSUPPORTED,
                   "weight type %d with in_dim %d: types 0, 1, 2, 12, 14 with in_dim a multiple "
                   "of 32 (of 256 for 12 and 14)",
                   type, in_dim);
  const uintptr_t need = (type == MIA_TYPE_Q4_0 || type == MIA_TYPE_Q6_K) ? 2 : 16;
  if ((uintptr_t)W & (need - 1))
    return set_err(MIA_ERR_INVALID, "W of type %d must be %d-byte aligned", type, (int)need);
  return MIA_OK;
}

// Y [S][N] (+)= X [S][K] . W^T for a weight type other than Q4_0, on fp16
// MFMA with fp32 accumulation (rocBLAS gemm_ex): X as fp16 hi + lo planes
// (launch_split_hilo), W as its fp16 values (Q4_K, F16: exact) or as row-scaled
// hi + lo planes (Q6_K, F32: launch_typed_split).  C1 = [Xhi; Xlo] . Whi^T in
// one GEMM of 2S columns, C2 = Xhi . Wlo^T; the combine kernel sums the parts
// (the Xlo . Wlo term, ~2^-22 of the product, is dropped).  rocBLAS is
// column-major: C^T [N][cols] = (W^T [K][N])^T . B^T [K][cols], so W is the
// transposed A operand with lda K and C's leading dimension is N.
static size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }

// The typed GEMM's packed form of a matrix of a type other than Q4_0: the fp16
// hi plane [N][K], then for Q6_K / F32 the lo plane [N][K] and the row scales
// [N] fp32, each at a 256-byte aligned offset (launch_typed_split's output).
static size_t typed_planes_bytes(int type, int N, int K) {
  const bool lo = !mia::typed_is_f16_exact(type);
  const size_t bw = al256((size_t)N * K * 2);
  return lo ? 2 * bw + al256((size_t)N * 4) : bw;
}

// reuse_x: split_work already holds X's planes (the call before split the
// same X on this stream), and X is not read.  packed: W is in the packed form
// (Q4_0: mia_q4_0_pack_gemm's tile layout; other types: the planes above).
static int typed_gemm_impl(DevCtx *c, const void *W, int type, const float *X, float *Y, int N,
                           int K, int S, bool add, hipStream_t s, bool reuse_x = false,
                           bool packed = false) {
  if (type == MIA_TYPE_Q4_0)
    return gemm_impl(c, W, nullptr, nullptr, N, 0, 0, X, K, S, Y, nullptr, nullptr,
                     add ? mia::kGemmAdd : mia::kGemmStore, s, reuse_x, nullptr, nullptr, packed);
  const bool lo = !mia::typed_is_f16_exact(type);
  const size_t bp = packed ? 0 : typed_planes_bytes(type, N, K);
  const size_t bc1 = al256((size_t)2 * S * N * 4), bc2 = al256((size_t)S * N * 4);
  if (int rc = ensure_wbuf(c, bp + bc1 + (lo ? bc2 : 0))) return rc;
  if (int rc = ensure_split_work(c, (size_t)2 * S * K * sizeof(_Float16))) return rc;
  if (int rc = ensure_lt(c)) return rc;
  char *w = reinterpret_cast<char *>(c->wbuf);
  char *planes = packed ? reinterpret_cast<char *>(const_cast<void *>(W)) : w;
  const size_t bw = al256((size_t)N * K * 2);
  _Float16 *whi = reinterpret_cast<_Float16 *>(planes);
  _Float16 *wlo = lo ? reinterpret_cast<_Float16 *>(planes + bw) : nullptr;
  float *rs = lo ? reinterpret_cast<float *>(planes + 2 * bw) : nullptr;
  float *C1 = reinterpret_cast<float *>(w + bp);
  float *C2 = lo ? reinterpret_cast<float *>(w + bp + bc1) : nullptr;
  _Float16 *xhi = reinterpret_cast<_Float16 *>(c->split_work);  // [2][S][K]: hi, then lo
  if (!packed) HIP_TRY(mia::launch_typed_split(W, type, whi, wlo, rs, N, K, s));
  if (!reuse_x)
    HIP_TRY(mia::launch_split_hilo(X, (long)S * K, xhi, xhi + (size_t)S * K, c->num_cus, s));
  if (int rc = lt_gemm(c, N, 2 * S, K, whi, xhi, C1, s)) return rc;
  if (lo)
    if (int rc = lt_gemm(c, N, S, K, wlo, xhi, C2, s)) return rc;
  HIP_TRY(mia::launch_hilo_combine(C1, C2, rs, Y, S, N, add, s));
  return MIA_OK;
}

long mia_weight_row_bytes(int type, int in_dim) { return mia::typed_row_bytes(type, in_dim); }

int mia_dequant_f32(const void *W, int type, float *out, int rows, int cols, void *stream) {
  if (!W || !out) return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (rows <= 0 || cols <= 0) return set_err(MIA_ERR_INVALID, "bad sizes (rows=%d cols=%d)", rows, cols);
  if (int rc = check_typed(type, cols, W)) return rc;
  if ((uintptr_t)out & 15) return set_err(MIA_ERR_INVALID, "out must be 16-byte aligned");
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  HIP_TRY(mia::launch_typed_dequant(W, type, out, rows, cols, pick_stream(c, stream)));
  return MIA_OK;
}

static int typed_matvec_impl(const void *W, int type, const void *x, bool xq8, float *y,
                             int out_dim, int in_dim, void *stream) {
  if (!W || !x || !y) return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (out_dim <= 0 || in_dim <= 0)
    return set_err(MIA_ERR_INVALID, "bad sizes (out_dim=%d in_dim=%d)", out_dim, in_dim);
  if (int rc = check_typed(type, in_dim, W)) return rc;
  if ((uintptr_t)x & (xq8 ? 3 : 15))
    return set_err(MIA_ERR_INVALID, "x must be %d-byte aligned", xq8 ? 4 : 16);
  if ((uintptr_t)y & 3) return set_err(MIA_ERR_INVALID, "y must be 4-byte aligned");
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  hipEvent_t ev0, ev1;
  if (int rc = prof_pair(c, 5, &ev0, &ev1)) return rc;
  HIP_TRY(mia::launch_typed_matvec(W, type, x, xq8, y, out_dim, in_dim, pick_stream(c, stream),
                                   ev0, ev1));
  return MIA_OK;
}

int mia_matvec_f32(const void *W, int type, const float *x, float *y, int out_dim, int in_dim,
                   void *stream) {
  return typed_matvec_impl(W, type, x, false, y, out_dim, in_dim, stream);
}

int mia_matvec_q8(const void *W, int type, const void *x_q8, float *y, int out_dim, int in_dim,
                  void *stream) {
  if (type == MIA_TYPE_Q4_0) return mia_q4_0_matvec(W, x_q8, y, out_dim, in_dim, stream);
  return typed_matvec_impl(W, type, x_q8, true, y, out_dim, in_dim, stream);
}

int mia_gemm_f32(const void *W, int type, const float *X, float *Y, int out_dim, int in_dim,
                 int S, void *stream) {
  if (type == MIA_TYPE_Q4_0) return mia_q4_0_gemm_f32(W, X, Y, out_dim, in_dim, S, stream);
  if (!W || !X || !Y) return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (out_dim <= 0 || in_dim <= 0 || S <= 0)
    return set_err(MIA_ERR_INVALID, "bad sizes (out_dim=%d in_dim=%d S=%d)", out_dim, in_dim, S);
  if (int rc = check_typed(type, in_dim, W)) return rc;
  if ((long)S * in_dim > INT_MAX || (long)S * out_dim > INT_MAX)
    return set_err(MIA_ERR_UNSUPPORTED, "S x dim above 2^31");
  if (int rc = check_align16(X, Y, nullptr, nullptr)) return rc;
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  return typed_gemm_impl(c, W, type, X, Y, out_dim, in_dim, S, false, pick_stream(c, stream));
}

static int typed_layer_impl(float *X, const mia_layer_weights_typed *lw, const float *theta_inv,
                            uint16_t *k_layer, uint16_t *v_layer, int dim, int hidden,
                            int n_heads, int n_kv_heads, float eps, int max_seq, int start_pos,
                            int S, void *stream, bool packed) {
  if (!lw) return set_err(MIA_ERR_INVALID, "NULL pointer");
  const int types[7] = {lw->wq_type, lw->wk_type, lw->wv_type, lw->wo_type,
                        lw->w1_type, lw->w2_type, lw->w3_type};
  bool all_q4_0 = true;
  for (int t : types) all_q4_0 = all_q4_0 && t == MIA_TYPE_Q4_0;
  if (all_q4_0) {
    const mia_layer_weights q{lw->wq, lw->wk, lw->wv, lw->wo, lw->w1,
                              lw->w2, lw->w3, lw->rms_att, lw->rms_ffn};
    return prefill_layer_impl(X, &q, theta_inv, k_layer, v_layer, dim, hidden, n_heads,
                              n_kv_heads, eps, max_seq, start_pos, S, stream, packed);
  }
  if (!X || !theta_inv || !k_layer || !v_layer) return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (!lw->wq || !lw->wk || !lw->wv || !lw->wo || !lw->w1 || !lw->w2 || !lw->w3 || !lw->rms_att ||
      !lw->rms_ffn)
    return set_err(MIA_ERR_INVALID, "NULL weight pointer");
  if (n_heads <= 0 || dim != n_heads * kHD)
    return set_err(MIA_ERR_UNSUPPORTED, "dim %d must be n_heads x 128", dim);
  if (int rc = check_shape(n_heads, n_kv_heads, kHD, max_seq)) return rc;
  if (int rc = check_pos(start_pos, S)) return rc;
  const int kv_dim = n_kv_heads * kHD;
  const void *const ws[7] = {lw->wq, lw->wk, lw->wv, lw->wo, lw->w1, lw->w2, lw->w3};
  const int in_dims[7] = {dim, dim, dim, dim, dim, hidden, dim};
  const int out_dims[7] = {dim, kv_dim, kv_dim, dim, hidden, dim, hidden};
  for (int i = 0; i < 7; ++i) {
    if (int rc = check_typed(types[i], in_dims[i], ws[i])) return rc;
    // Q4_0 matrices take the fp16-MFMA GEMM (4-byte aligned, in_dim a multiple of 64)
    if (types[i] == MIA_TYPE_Q4_0) {
      if (in_dims[i] % 64) return set_err(MIA_ERR_UNSUPPORTED, "Q4_0 GEMM needs in_dim %% 64 == 0");
      if ((uintptr_t)ws[i] & 3) return set_err(MIA_ERR_INVALID, "Q4_0 weights must be 4-byte aligned");
    }
    if (packed && ((uintptr_t)ws[i] & 15))
      return set_err(MIA_ERR_INVALID, "packed weights must be 16-byte aligned");
    if (packed && types[i] == MIA_TYPE_Q4_0 && out_dims[i] % 64)
      return set_err(MIA_ERR_UNSUPPORTED, "packed Q4_0 needs out_dim %% 64 == 0");
  }
  if (hidden <= 0 || (long)S * hidden > INT_MAX || (long)S * dim > INT_MAX)
    return set_err(MIA_ERR_UNSUPPORTED, "bad hidden %d or S x dim above 2^31", hidden);
  if (int rc = check_align16(X, lw->rms_att, lw->rms_ffn, k_layer)) return rc;
  if (int rc = check_align16(v_layer, nullptr, nullptr, nullptr)) return rc;
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  hipStream_t s = pick_stream(c, stream);
  // XN, Q, A [S][dim] | K, V [S][kv_dim] | G, U [S][hidden], all fp32
  auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
  const size_t bd = al((size_t)S * dim * 4), bk = al((size_t)S * kv_dim * 4),
               bh = al((size_t)S * hidden * 4);
  if (int rc = ensure_layer_work(c, 3 * bd + 2 * bk + 2 * bh)) return rc;
  char *w = reinterpret_cast<char *>(c->layer_work);
  float *XN = reinterpret_cast<float *>(w);
  float *Q = reinterpret_cast<float *>(w + bd);
  float *A = reinterpret_cast<float *>(w + 2 * bd);
  float *K = reinterpret_cast<float *>(w + 3 * bd);
  float *V = reinterpret_cast<float *>(w + 3 * bd + bk);
  float *G = reinterpret_cast<float *>(w + 3 * bd + 2 * bk);
  float *U = reinterpret_cast<float *>(w + 3 * bd + 2 * bk + bh);
  // mistral_ane_prefill.h:1092-1110
  HIP_TRY(mia::launch_rmsnorm(XN, X, lw->rms_att, dim, S, eps, s));
  // (the normalised rows are split into fp16 planes once for Q, K and V)
  if (int rc = typed_gemm_impl(c, lw->wq, lw->wq_type, XN, Q, dim, dim, S, false, s, false, packed))
    return rc;
  if (int rc = typed_gemm_impl(c, lw->wk, lw->wk_type, XN, K, kv_dim, dim, S, false, s, true, packed))
    return rc;
  if (int rc = typed_gemm_impl(c, lw->wv, lw->wv_type, XN, V, kv_dim, dim, S, false, s, true, packed))
    return rc;
  // apply_rope_batch, kv_write_batch, attention_batch, as mia_prefill_layer
  if (int rc = ensure_work(c, (size_t)S * kHD * sizeof(float))) return rc;
  float *cs = reinterpret_cast<float *>(c->work);
  HIP_TRY(mia::launch_rope_to_ring(K, V, theta_inv, S, start_pos, n_kv_heads,
                                   reinterpret_cast<_Float16 *>(k_layer),
                                   reinterpret_cast<_Float16 *>(v_layer), max_seq, cs, s));
  if (int rc = flash_impl(c, Q, cs, nullptr, nullptr, k_layer, v_layer, A, n_kv_heads, max_seq,
                          start_pos, S, s))
    return rc;
  // X + A . Wo^T (vDSP_vadd after the GEMM: the sum rounded once more)
  if (int rc = typed_gemm_impl(c, lw->wo, lw->wo_type, A, X, dim, dim, S, true, s, false, packed))
    return rc;
  HIP_TRY(mia::launch_rmsnorm(XN, X, lw->rms_ffn, dim, S, eps, s));
  if (int rc = typed_gemm_impl(c, lw->w1, lw->w1_type, XN, G, hidden, dim, S, false, s, false, packed))
    return rc;
  if (int rc = typed_gemm_impl(c, lw->w3, lw->w3_type, XN, U, hidden, dim, S, false, s, true, packed))
    return rc;
  HIP_TRY(mia::launch_silu_mul(G, U, (long)S * hidden, s));
  return typed_gemm_impl(c, lw->w2, lw->w2_type, G, X, dim, hidden, S, true, s, false, packed);
}

int mia_prefill_layer_typed(float *X, const mia_layer_weights_typed *lw, const float *theta_inv,
                            uint16_t *k_layer, uint16_t *v_layer, int dim, int hidden,
                            int n_heads, int n_kv_heads, float eps, int max_seq, int start_pos,
                            int S, void *stream) {
  return typed_layer_impl(X, lw, theta_inv, k_layer, v_layer, dim, hidden, n_heads, n_kv_heads,
                          eps, max_seq, start_pos, S, stream, false);
}

int mia_prefill_layer_typed_packed(float *X, const mia_layer_weights_typed *lw,
                                   const float *theta_inv, uint16_t *k_layer, uint16_t *v_layer,
                                   int dim, int hidden, int n_heads, int n_kv_heads, float eps,
                                   int max_seq, int start_pos, int S, void *stream) {
  return typed_layer_impl(X, lw, theta_inv, k_layer, v_layer, dim, hidden, n_heads, n_kv_heads,
                          eps, max_seq, start_pos, S, stream, true);
}

size_t mia_gemm_pack_bytes(int type, int out_dim, int in_dim) {
  if (out_dim <= 0 || mia::typed_row_bytes(type, in_dim) == 0) return 0;
  if (type == MIA_TYPE_Q4_0)
    return (out_dim % 64 || in_dim % 64) ? 0 : (size_t)out_dim * (in_dim / 32) * 18;
  return typed_planes_bytes(type, out_dim, in_dim);
}

int mia_gemm_pack(const void *W, int type, void *Wp, int out_dim, int in_dim, void *stream) {
  if (type == MIA_TYPE_Q4_0) return mia_q4_0_pack_gemm(W, Wp, out_dim, in_dim, stream);
  if (!W || !Wp) return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (out_dim <= 0) return set_err(MIA_ERR_INVALID, "bad out_dim %d", out_dim);
  if (int rc = check_typed(type, in_dim, W)) return rc;
  if ((uintptr_t)Wp & 15) return set_err(MIA_ERR_INVALID, "Wp must be 16-byte aligned");
  const size_t nb = typed_planes_bytes(type, out_dim, in_dim);
  const uintptr_t wb = (uintptr_t)out_dim * (uintptr_t)mia::typed_row_bytes(type, in_dim);
  const uintptr_t a = (uintptr_t)W, b = (uintptr_t)Wp;
  if (a < b + nb && b < a + wb) return set_err(MIA_ERR_INVALID, "W and Wp overlap");
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  char *p = reinterpret_cast<char *>(Wp);
  const size_t bw = al256((size_t)out_dim * in_dim * 2);
  const bool lo = !mia::typed_is_f16_exact(type);
  HIP_TRY(mia::launch_typed_split(W, type, reinterpret_cast<_Float16 *>(p),
                                  lo ? reinterpret_cast<_Float16 *>(p + bw) : nullptr,
                                  lo ? reinterpret_cast<float *>(p + 2 * bw) : nullptr, out_dim,
                                  in_dim, pick_stream(c, stream)));
  return MIA_OK;
}

int mia_gemm_packed_f32(const void *Wp, int type, const float *X, float *Y, int out_dim,
                        int in_dim, int S, void *stream) {
  if (type == MIA_TYPE_Q4_0)
    return mia_q4_0_gemm_packed_f32(Wp, X, Y, out_dim, in_dim, S, stream);
  if (!Wp || !X || !Y) return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (out_dim <= 0 || in_dim <= 0 || S <= 0)
    return set_err(MIA_ERR_INVALID, "bad sizes (out_dim=%d in_dim=%d S=%d)", out_dim, in_dim, S);
  if (mia::typed_row_bytes(type, in_dim) == 0)
    return set_err(MIA_ERR_UNSUPPORTED, "weight type %d with in_dim %d", type, in_dim);
  if ((uintptr_t)Wp & 15) return set_err(MIA_ERR_INVALID, "Wp must be 16-byte aligned");
  if ((long)S * in_dim > INT_MAX || (long)S * out_dim > INT_MAX)
    return set_err(MIA_ERR_UNSUPPORTED, "S x dim above 2^31");
  if (int rc = check_align16(X, Y, nullptr, nullptr)) return rc;
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  return typed_gemm_impl(c, Wp, type, X, Y, out_dim, in_dim, S, false, pick_stream(c, stream),
                         false, true);
}

int mia_quantize_q8_0(const float *x, void *out_q8, int n, void *stream) {
  if (!x || !out_q8) return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (n <= 0 || n % 32) return set_err(MIA_ERR_INVALID, "n %d must be a positive multiple of 32", n);
  if ((uintptr_t)x & 15) return set_err(MIA_ERR_INVALID, "x must be 16-byte aligned");
  if ((uintptr_t)out_q8 & 3) return set_err(MIA_ERR_INVALID, "out_q8 must be 4-byte aligned");
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  HIP_TRY(mia::launch_quantize_q8_0(x, reinterpret_cast<uint8_t *>(out_q8), n / 32,
                                    pick_stream(c, stream)));
  return MIA_OK;
}

int mia_q4_0_matvec(const void *W, const void *x_q8, float *y, int out_dim, int in_dim,
                    void *stream) {
  return q4_impl(W, nullptr, nullptr, x_q8, nullptr, y, nullptr, nullptr, out_dim, 0, in_dim,
                 stream);
}

int mia_q4_0_matvec_qkv(const void *Wq, const void *Wk, const void *Wv, const void *x_q8,
                        float *yq, float *yk, float *yv, int dim, int kv_dim, int in_dim,
                        void *stream) {
  return q4_impl(Wq, Wk, Wv, x_q8, nullptr, yq, yk, yv, dim, kv_dim, in_dim, stream);
}

int mia_q4_0_matvec_f32(const void *W, const float *x, float *y, int out_dim, int in_dim,
                        void *stream) {
  return q4_impl(W, nullptr, nullptr, nullptr, x, y, nullptr, nullptr, out_dim, 0, in_dim, stream);
}

int mia_q4_0_matvec_qkv_f32(const void *Wq, const void *Wk, const void *Wv, const float *x,
                            float *yq, float *yk, float *yv, int dim, int kv_dim, int in_dim,
                            void *stream) {
  return q4_impl(Wq, Wk, Wv, nullptr, x, yq, yk, yv, dim, kv_dim, in_dim, stream);
}

// Two matrices of out_dim rows against one input: W1 (gate) and W3 (up) of
// the FFN, mistral_model.h:750-811.
static int q4_pair_impl(const void *W1, const void *W3, const void *x_q8, const float *xf,
                        float *y1, float *y3, int out_dim, int in_dim, void *stream) {
  if (!W1 || !W3 || !(x_q8 || xf) || !y1 || !y3) return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (out_dim <= 0 || in_dim <= 0 || in_dim % 32 || out_dim > INT_MAX / 2)
    return set_err(MIA_ERR_INVALID, "bad sizes (out_dim=%d in_dim=%d)", out_dim, in_dim);
  if (in_dim % 64)
    return set_err(MIA_ERR_UNSUPPORTED, "in_dim %d: the kernel needs an even number of blocks per row",
                   in_dim);
  if (xf && in_dim > mia::kQ4MaxF32InDim)
    return set_err(MIA_ERR_UNSUPPORTED, "in_dim %d above %d for fp32 input (quantize first)", in_dim,
                   mia::kQ4MaxF32InDim);
  const uintptr_t bits = (uintptr_t)W1 | (uintptr_t)W3 | (uintptr_t)x_q8 | (uintptr_t)y1 |
                         (uintptr_t)y3;
  if (bits & 3) return set_err(MIA_ERR_INVALID, "weights, x_q8 and y must be 4-byte aligned");
  if ((uintptr_t)xf & 15) return set_err(MIA_ERR_INVALID, "x must be 16-byte aligned");
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  mia::Q4MatvecParams p{};
  p.w0 = reinterpret_cast<const uint8_t *>(W1);
  p.w1 = reinterpret_cast<const uint8_t *>(W3);
  p.y0 = y1;
  p.y1 = y3;
  p.x = reinterpret_cast<const uint8_t *>(x_q8);
  p.xf = xf;
  p.rows0 = out_dim;
  p.rows01 = 2 * out_dim;
  p.total_rows = 2 * out_dim;
  p.bpr = in_dim / 32;
  hipEvent_t ev0, ev1;
  if (int rc = prof_pair(c, 2, &ev0, &ev1)) return rc;
  HIP_TRY(mia::launch_q4_matvec(p, pick_stream(c, stream), ev0, ev1));
  return MIA_OK;
}

int mia_q4_0_matvec_pair(const void *W1, const void *W3, const void *x_q8, float *y1, float *y3,
                         int out_dim, int in_dim, void *stream) {
  return q4_pair_impl(W1, W3, x_q8, nullptr, y1, y3, out_dim, in_dim, stream);
}

int mia_q4_0_matvec_pair_f32(const void *W1, const void *W3, const float *x, float *y1,
                             float *y3, int out_dim, int in_dim, void *stream) {
  return q4_pair_impl(W1, W3, nullptr, x, y1, y3, out_dim, in_dim, stream);
}

// ---- the decode layer -------------------------------------------------------

// y [rows] = W . x for the layer's matrices on Q8_0 input blocks, by type as
// q4_matvec_sdot_parallel dispatches (mistral_model.h:649-670).
static int layer_matvec_q8(const void *W, int type, const void *xq8, float *y, int rows, int cols,
                           void *stream) {
  if (type == MIA_TYPE_Q4_0) return mia_q4_0_matvec(W, xq8, y, rows, cols, stream);
  return typed_matvec_impl(W, type, xq8, true, y, rows, cols, stream);
}

int mia_silu_mul_f32(float *gate, const float *up, long n, void *stream) {
  if (!gate || !up) return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (n < 0) return set_err(MIA_ERR_INVALID, "bad size %ld", n);
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  HIP_TRY(mia::launch_silu_mul(gate, up, n, pick_stream(c, stream)));
  return MIA_OK;
}

int mia_decode_layer(float *x, const mia_layer_weights_typed *lw, const float *theta_inv,
                     uint16_t *k_layer, uint16_t *v_layer, int dim, int hidden, int n_heads,
                     int n_kv_heads, float eps, int max_seq, int pos, void *stream) {
  if (!x || !lw || !theta_inv || !k_layer || !v_layer)
    return set_err(MIA_ERR_INVALID, "NULL pointer");
  if (!lw->wq || !lw->wk || !lw->wv || !lw->wo || !lw->w1 || !lw->w2 || !lw->w3 || !lw->rms_att ||
      !lw->rms_ffn)
    return set_err(MIA_ERR_INVALID, "NULL weight pointer");
  if (n_heads <= 0 || dim != n_heads * kHD)
    return set_err(MIA_ERR_UNSUPPORTED, "dim %d must be n_heads x 128", dim);
  if (int rc = check_shape(n_heads, n_kv_heads, kHD, max_seq)) return rc;
  if (int rc = check_pos(pos, 1)) return rc;
  if (hidden <= 0) return set_err(MIA_ERR_INVALID, "bad hidden %d", hidden);
  const int kv_dim = n_kv_heads * kHD;
  const void *const ws[7] = {lw->wq, lw->wk, lw->wv, lw->wo, lw->w1, lw->w2, lw->w3};
  const int types[7] = {lw->wq_type, lw->wk_type, lw->wv_type, lw->wo_type,
                        lw->w1_type, lw->w2_type, lw->w3_type};
  const int in_dims[7] = {dim, dim, dim, dim, dim, hidden, dim};
  for (int i = 0; i < 7; ++i) {
    if (int rc = check_typed(types[i], in_dims[i], ws[i])) return rc;
    if (types[i] == MIA_TYPE_Q4_0) {  // the W4A8 kernel: whole block pairs, 4-byte aligned
      if (in_dims[i] % 64)
        return set_err(MIA_ERR_UNSUPPORTED, "Q4_0 matvec needs in_dim %% 64 == 0");
      if ((uintptr_t)ws[i] & 3)
        return set_err(MIA_ERR_INVALID, "Q4_0 weights must be 4-byte aligned");
    }
  }
  if (int rc = check_align16(x, lw->rms_att, lw->rms_ffn, nullptr)) return rc;
  DevCtx *c;
  if (int rc = current_ctx(&c)) return rc;
  hipStream_t s = pick_stream(c, stream);
  // xb, xb2, q [dim] | k, v [kv_dim] | hb, hb2 [hidden] | Q8_0 blocks of the
  // longest input
  const size_t bd = al256((size_t)dim * 4), bk = al256((size_t)kv_dim * 4),
               bh = al256((size_t)hidden * 4),
               bq = al256((size_t)(dim > hidden ? dim : hidden) / 32 * 36);
  if (int rc = ensure_dl_work(c, 3 * bd + 2 * bk + 2 * bh + bq)) return rc;
  char *w = reinterpret_cast<char *>(c->dl_work);
  float *xb = reinterpret_cast<float *>(w);
  float *xb2 = reinterpret_cast<float *>(w + bd);
  float *q = reinterpret_cast<float *>(w + 2 * bd);
  float *k = reinterpret_cast<float *>(w + 3 * bd);
  float *v = reinterpret_cast<float *>(w + 3 * bd + bk);
  float *hb = reinterpret_cast<float *>(w + 3 * bd + 2 * bk);
  float *hb2 = reinterpret_cast<float *>(w + 3 * bd + 2 * bk + bh);
  void *q8 = w + 3 * bd + 2 * bk + 2 * bh;
  const bool fused_in = dim <= mia::kQ4MaxF32InDim;  // x quantised inside the Q4_0 launch
  bool all_q4_0 = true;
  for (int t : types) all_q4_0 = all_q4_0 && t == MIA_TYPE_Q4_0;
  if (all_q4_0 && fused_in && hidden <= mia::kQ4MaxFusedInDim) {
    // mistral_model.h:830-899 in four matvec launches around the attention:
    // each RMSNorm and Q8_0 quantisation happens in the prologue of the
    // matvec that reads it, each residual add and the SwiGLU product in the
    // epilogue of the matvec that produces them; the arithmetic is that of
    // the separate steps, bit for bit.
    auto mv = [&](const void *w0, const void *w1, const void *w2, float *y0, float *y1,
                  float *y2, int rows0, int rows1, int rows2, const float *xf, int in_dim,
                  const float *rms_w, const float *up, const float *resid,
                  bool swiglu = false) -> int {
      mia::Q4MatvecParams p{};
      p.w0 = reinterpret_cast<const uint8_t *>(w0);
      p.w1 = reinterpret_cast<const uint8_t *>(w1);
      p.w2 = reinterpret_cast<const uint8_t *>(w2);
      p.y0 = y0;
      p.y1 = y1;
      p.y2 = y2;
      p.xf = xf;
      p.rows0 = rows0;
      p.rows01 = rows0 + rows1;
      p.total_rows = rows0 + rows1 + rows2;
      p.bpr = in_dim / 32;
      p.rms_w = rms_w;
      p.eps = eps;
      p.up = up;
      p.resid = resid;
      p.swiglu = swiglu ? 1 : 0;
      hipEvent_t ev0, ev1;
      if (int rc = prof_pair(c, 2, &ev0, &ev1)) return rc;
      HIP_TRY(mia::launch_q4_matvec(p, s, ev0, ev1));
      return MIA_OK;
    };
    if (int rc = mv(lw->wq, lw->wk, lw->wv, q, k, v, dim, kv_dim, kv_dim, x, dim, lw->rms_att,
                    nullptr, nullptr))
      return rc;
    if (int rc = decode_impl(q, k, v, theta_inv, k_layer, v_layer, xb2, n_heads, n_kv_heads,
                             max_seq, pos, true, s))
      return rc;
    if (int rc = mv(lw->wo, nullptr, nullptr, x, nullptr, nullptr, dim, 0, 0, xb2, dim, nullptr,
                    nullptr, x))
      return rc;
    // gate and up rows interleaved: each wave ends with its row's SwiGLU product
    if (int rc = mv(lw->w1, lw->w3, nullptr, hb, nullptr, nullptr, hidden, hidden, 0, x, dim,
                    lw->rms_ffn, nullptr, nullptr, true))
      return rc;
    return mv(lw->w2, nullptr, nullptr, x, nullptr, nullptr, dim, 0, 0, hb, hidden, nullptr,
              nullptr, x);
  }
  bool all_kquant = types[4] == types[6];
  for (int t : types) all_kquant = all_kquant && (t == MIA_TYPE_Q4_K || t == MIA_TYPE_Q6_K);
  if (all_kquant && dim <= mia::kKqLayerMaxCols && hidden <= mia::kKqLayerMaxCols) {
    // The same four matvec launches around the attention with Q4_K / Q6_K
    // weights (Q4_K_M and its like): each forms its input's Q8_0 blocks, after
    // the RMSNorm where there is one, in its prologue.
    auto kl = [&](const void *w0, const void *w1, const void *w2, int t0, int t1, int t2,
                  float *y0, float *y1, float *y2, int r0, int r1, int r2, const float *xf,
                  int cols, const float *rms_w, const float *resid, bool swiglu) -> int {
      mia::KqLayerParams p{};
      p.w[0] = w0;
      p.w[1] = w1;
      p.w[2] = w2;
      p.type[0] = t0;
      p.type[1] = t1;
      p.type[2] = t2;
      p.y[0] = y0;
      p.y[1] = y1;
      p.y[2] = y2;
      p.rows[0] = r0;
      p.rows[1] = r1;
      p.rows[2] = r2;
      p.cols = cols;
      p.xf = xf;
      p.rms_w = rms_w;
      p.eps = eps;
      p.resid = resid;
      p.swiglu = swiglu ? 1 : 0;
      hipEvent_t ev0, ev1;
      if (int rc = prof_pair(c, 5, &ev0, &ev1)) return rc;
      HIP_TRY(mia::launch_kq_layer_matvec(p, s, ev0, ev1));
      return MIA_OK;
    };
    if (int rc = kl(lw->wq, lw->wk, lw->wv, types[0], types[1], types[2], q, k, v, dim, kv_dim,
                    kv_dim, x, dim, lw->rms_att, nullptr, false))
      return rc;
    if (int rc = decode_impl(q, k, v, theta_inv, k_layer, v_layer, xb2, n_heads, n_kv_heads,
                             max_seq, pos, true, s))
      return rc;
    if (int rc = kl(lw->wo, nullptr, nullptr, types[3], 0, 0, x, nullptr, nullptr, dim, 0, 0, xb2,
                    dim, nullptr, x, false))
      return rc;
    if (int rc = kl(lw->w1, lw->w3, nullptr, types[4], types[6], 0, hb, nullptr, nullptr, hidden,
                    hidden, 0, x, dim, lw->rms_ffn, nullptr, true))
      return rc;
    return kl(lw->w2, nullptr, nullptr, types[5], 0, 0, x, nullptr, nullptr, dim, 0, 0, hb, hidden,
              nullptr, x, false);
  }
  // mistral_model.h:830-899
  HIP_TRY(mia::launch_rmsnorm(xb, x, lw->rms_att, dim, 1, eps, s));
  if (types[0] == MIA_TYPE_Q4_0 && types[1] == MIA_TYPE_Q4_0 && types[2] == MIA_TYPE_Q4_0 &&
      fused_in) {
    if (int rc = mia_q4_0_matvec_qkv_f32(lw->wq, lw->wk, lw->wv, xb, q, k, v, dim, kv_dim, dim, s))
      return rc;
  } else {
    HIP_TRY(mia::launch_quantize_q8_0(xb, reinterpret_cast<uint8_t *>(q8), dim / 32, s));
    if (int rc = layer_matvec_q8(lw->wq, types[0], q8, q, dim, dim, s)) return rc;
    if (int rc = layer_matvec_q8(lw->wk, types[1], q8, k, kv_dim, dim, s)) return rc;
    if (int rc = layer_matvec_q8(lw->wv, types[2], q8, v, kv_dim, dim, s)) return rc;
  }
  // RoPE, fp16 ring write at pos % max_seq, attention: one fused launch + merge
  if (int rc = decode_impl(q, k, v, theta_inv, k_layer, v_layer, xb2, n_heads, n_kv_heads, max_seq,
                           pos, true, s))
    return rc;
  if (types[3] == MIA_TYPE_Q4_0 && fused_in) {
    if (int rc = mia_q4_0_matvec_f32(lw->wo, xb2, xb, dim, dim, s)) return rc;
  } else {
    HIP_TRY(mia::launch_quantize_q8_0(xb2, reinterpret_cast<uint8_t *>(q8), dim / 32, s));
    if (int rc = layer_matvec_q8(lw->wo, types[3], q8, xb, dim, dim, s)) return rc;
  }
  HIP_TRY(mia::launch_residual_rmsnorm(x, xb, lw->rms_ffn, xb, dim, eps, s));
  if (types[4] == MIA_TYPE_Q4_0 && types[6] == MIA_TYPE_Q4_0 && fused_in) {
    if (int rc = mia_q4_0_matvec_pair_f32(lw->w1, lw->w3, xb, hb, hb2, hidden, dim, s)) return rc;
  } else {
    HIP_TRY(mia::launch_quantize_q8_0(xb, reinterpret_cast<uint8_t *>(q8), dim / 32, s));
    if (int rc = layer_matvec_q8(lw->w1, types[4], q8, hb, hidden, dim, s)) return rc;
    if (int rc = layer_matvec_q8(lw->w3, types[6], q8, hb2, hidden, dim, s)) return rc;
  }
  HIP_TRY(mia::launch_silu_mul(hb, hb2, hidden, s));
  HIP_TRY(mia::launch_quantize_q8_0(hb, reinterpret_cast<uint8_t *>(q8), hidden / 32, s));
  if (int rc = layer_matvec_q8(lw->w2, types[5], q8, xb, dim, hidden, s)) return rc;
  HIP_TRY(mia::launch_add(x, xb, dim, s));
  return MIA_OK;
}

}  // extern "C"
