// extern "C" entry points of libflexatt (declared in include/flexatt.h):
// argument checks, then dispatch to the kernel launchers by dtype and head dim.
#include <math.h>
#include <stdint.h>

#include <atomic>
#include <mutex>

#include "../../include/flexatt.h"
#include "flexatt_kernels.h"

namespace {
using namespace flexatt;

size_t elt_size(int dt) {
  switch (dt) {
    case FLEXATT_F32: return 4;
    case FLEXATT_F16:
    case FLEXATT_BF16: return 2;
    default: return 0;
  }
}

int head_index(int d) {
  switch (d) {
    case 32: return 0;
    case 64: return 1;
    case 128: return 2;
    case 256: return 3;
    default: return -1;
  }
}

int check_problem(const flexatt_problem* p) {
  if (!p) return FLEXATT_EINVAL;
  if (elt_size(p->dtype) == 0) return FLEXATT_EDTYPE;
  if (p->batch <= 0 || p->heads_q <= 0 || p->heads_kv <= 0 || p->seqlen_q <= 0 || p->seqlen_kv <= 0)
    return FLEXATT_EINVAL;
  if (p->heads_q % p->heads_kv != 0) return FLEXATT_ESHAPE;
  if (p->doc_bounds && !p->col_bounds && p->seqlen_q != p->seqlen_kv) return FLEXATT_ESHAPE;
  if (p->col_bounds && !p->doc_bounds) return FLEXATT_EINVAL;
  if (p->reserved != 0) return FLEXATT_EINVAL;
  if (p->block_map) {
    if (p->block_heads != 1 && p->block_heads != p->heads_q) return FLEXATT_EINVAL;
    if ((p->seqlen_kv + kBlk - 1) / kBlk > kBlkRowMax) return FLEXATT_ERANGE;
  }
  if (head_index(p->head_dim) < 0) return FLEXATT_EHEADDIM;
  if (p->causal != 0 && p->causal != 1) return FLEXATT_EINVAL;
  if (p->sliding_window < 0) return FLEXATT_EINVAL;
  if (!(p->soft_cap >= 0.f) || !isfinite(p->soft_cap) || !isfinite(p->scale)) return FLEXATT_EINVAL;
  // Grid sizes: tiles * B * H must fit a 1-D grid; row counts fit int32.
  const int64_t rows_q = (int64_t)p->batch * p->heads_q * p->seqlen_q;
  const int64_t rows_k = (int64_t)p->batch * p->heads_kv * p->seqlen_kv;
  if (rows_q > INT32_MAX || rows_k > INT32_MAX) return FLEXATT_ESHAPE;
  return FLEXATT_OK;
}

#define FLEXATT_TRY_OK(x)               \
  do {                                  \
    const int rc_ = (x);                \
    if (rc_ != FLEXATT_OK) return rc_;  \
  } while (0)

int check_tensor(const flexatt_tensor* t, int dt) {
  if (!t || !t->data) return FLEXATT_EINVAL;
  const int64_t es = (int64_t)elt_size(dt);
  if (t->stride_d != 1) return FLEXATT_ELAYOUT;
  if (t->stride_b < 0 || t->stride_h < 0 || t->stride_s < 0) return FLEXATT_ELAYOUT;
  if (((uintptr_t)t->data) % 16 != 0) return FLEXATT_ELAYOUT;
  if ((t->stride_b * es) % 16 || (t->stride_h * es) % 16 || (t->stride_s * es) % 16) return FLEXATT_ELAYOUT;
  return FLEXATT_OK;
}

// Output tensors: the input rules, and no two elements of the [b, h, s, d]
// index space may share an address (several workgroups would store to it,
// and the results would depend on their order).  Sufficient test: over the
// dimensions of extent > 1 sorted by stride, each stride exceeds the span of
// the smaller ones.
int check_out_tensor(const flexatt_tensor* t, int dt, int64_t n_b, int64_t n_h, int64_t n_s, int64_t n_d) {
  FLEXATT_TRY_OK(check_tensor(t, dt));
  int64_t st[4] = {t->stride_b, t->stride_h, t->stride_s, 1};
  int64_t ext[4] = {n_b, n_h, n_s, n_d};
  int order[4], n = 0;
  for (int i = 0; i < 4; ++i)
    if (ext[i] > 1) order[n++] = i;
  for (int i = 1; i < n; ++i)  // insertion sort by stride
    for (int j = i; j > 0 && st[order[j]] < st[order[j - 1]]; --j) {
      const int x = order[j];
      order[j] = order[j - 1];
      order[j - 1] = x;
    }
  int64_t span = 0;  // largest offset reachable with the dims sorted so far
  for (int i = 0; i < n; ++i) {
    const int d = order[i];
    if (st[d] <= span) return FLEXATT_ELAYOUT;
    span += (ext[d] - 1) * st[d];
  }
  return FLEXATT_OK;
}

Shape make_shape(const flexatt_problem* p) {
  Shape s;
  s.B = p->batch;
  s.Hq = p->heads_q;
  s.Hkv = p->heads_kv;
  s.G = p->heads_q / p->heads_kv;
  s.Sq = p->seqlen_q;
  s.Skv = p->seqlen_kv;
  s.scale = p->scale;
  s.scale_log2 = p->scale * kLog2e;
  s.causal = p->causal;
  s.window = p->sliding_window;
  s.cap = p->soft_cap;
  s.inv_cap = p->soft_cap > 0.f ? 1.0f / p->soft_cap : 0.f;
  s.tanh_k = p->soft_cap > 0.f ? 2.0f * kLog2e * p->scale / p->soft_cap : 0.f;
  s.cap_log2 = p->soft_cap * kLog2e;
  s.alibi = p->alibi_slopes;
  s.doc = p->doc_bounds;
  s.docc = p->col_bounds ? p->col_bounds : p->doc_bounds;
  s.blk = p->block_map;
  s.blk_h = p->block_map ? p->block_heads : 1;
  s.blk_nq = (p->seqlen_q + kBlk - 1) / kBlk;
  s.blk_nk = (p->seqlen_kv + kBlk - 1) / kBlk;
  return s;
}

View view(const flexatt_tensor* t) { return View{t->data, t->stride_b, t->stride_h, t->stride_s}; }
MutView mview(const flexatt_tensor* t) { return MutView{t->data, t->stride_b, t->stride_h, t->stride_s}; }

// [dtype][head index]
const FwdLauncher kFwd[3][4] = {
    {fwd_f32_d32, fwd_f32_d64, fwd_f32_d128, fwd_f32_d256},
    {fwd_mfma_f16_d32, fwd_mfma_f16_d64, fwd_mfma_f16_d128, fwd_mfma_f16_d256},
    {fwd_mfma_bf16_d32, fwd_mfma_bf16_d64, fwd_mfma_bf16_d128, fwd_mfma_bf16_d256},
};
const BwdLauncher kDq[3][4] = {
    {bwd_dq_f32_d32, bwd_dq_f32_d64, bwd_dq_f32_d128, bwd_dq_f32_d256},
    {bwd_dq_mfma_f16_d32, bwd_q_f16_d64, bwd_q_f16_d128, bwd_dq_mfma_f16_d256},
    {bwd_dq_mfma_bf16_d32, bwd_q_bf16_d64, bwd_q_bf16_d128, bwd_dq_mfma_bf16_d256},
};
const BwdLauncher kDkdv[3][4] = {
    {bwd_dkdv_f32_d32, bwd_dkdv_f32_d64, bwd_dkdv_f32_d128, bwd_dkdv_f32_d256},
    {bwd_dkdv_mfma_f16_d32, bwd_kv_f16_d64, bwd_kv_f16_d128, bwd_kv_f16_d256},
    {bwd_dkdv_mfma_bf16_d32, bwd_kv_bf16_d64, bwd_kv_bf16_d128, bwd_kv_bf16_d256},
};

// Split-KV decode: range, plan and workspace.
constexpr int kDecWaves = 4;  // waves per workgroup
constexpr int kDecTile = 32;   // KV rows per tile
bool decode_applies(const flexatt_problem* p) {
  return (p->dtype == FLEXATT_F16 || p->dtype == FLEXATT_BF16) && p->head_dim <= 128 && !p->doc_bounds &&
         !p->block_map &&
         (int64_t)(p->heads_q / p->heads_kv) * p->seqlen_q <= 32;
}
struct DecodePlan {
  int nsplit, chunk, ntiles;
  size_t bytes;  // workspace: partial O then partial LSE
};
DecodePlan decode_plan(const flexatt_problem* p) {
  DecodePlan d;
  // attended KV range: with top-left causal alignment no query row sees past Sq - 1
  const int kv_hi = p->causal ? (p->seqlen_kv < p->seqlen_q ? p->seqlen_kv : p->seqlen_q) : p->seqlen_kv;
  d.ntiles = (kv_hi + kDecTile - 1) / kDecTile;
  // about two workgroups per CU (256 CUs), but at least two tiles per wave
  const int64_t groups = (int64_t)p->batch * p->heads_kv;
  int64_t ns = (512 + groups - 1) / groups;
  const int64_t most = d.ntiles / (2 * kDecWaves);
  if (ns > most) ns = most;
  if (ns > 256) ns = 256;
  if (ns < 1) ns = 1;
  d.chunk = (int)((d.ntiles + ns - 1) / ns);
  d.nsplit = (d.ntiles + d.chunk - 1) / d.chunk;  // no workgroup without tiles
  const int64_t rows = (int64_t)p->batch * p->heads_q * p->seqlen_q;
  const int64_t parts = d.nsplit;  // one partial per workgroup
  d.bytes = (size_t)(rows * parts * (p->head_dim + 1) * (int64_t)sizeof(float));
  return d;
}
const DecodeLauncher kDecode[3][3] = {
    {nullptr, nullptr, nullptr},
    {fwd_decode_f16_d32, fwd_decode_f16_d64, fwd_decode_f16_d128},
    {fwd_decode_bf16_d32, fwd_decode_bf16_d64, fwd_decode_bf16_d128},
};

// Launch the decode kernels with their partials in `ws` (d.bytes, 16-byte
// aligned); the problem and tensors are already checked.
int decode_run(const flexatt_problem* p, const DecodePlan& d, const flexatt_tensor* q, const flexatt_tensor* k,
               const flexatt_tensor* v, const flexatt_tensor* o, float* lse, void* ws, hipStream_t stream) {
  DecodeArgs a;
  a.q = view(q);
  a.k = view(k);
  a.v = view(v);
  a.o = mview(o);
  a.lse = lse;
  a.p = make_shape(p);
  a.nsplit = d.nsplit;
  a.chunk = d.chunk;
  a.ntiles = d.ntiles;
  const int64_t rows = (int64_t)p->batch * p->heads_q * p->seqlen_q;
  a.part_o = (float*)ws;
  a.part_lse = a.part_o + rows * d.nsplit * p->head_dim;
  return (int)kDecode[p->dtype][head_index(p->head_dim)](a, stream);
}

// Fixed partial-result buffer of flexatt_fwd_decode_noalloc: one copy per GPU,
// held until the process ends.  Host code never passes the name `scratch`
// itself to a kernel (on the host it is a stand-in, not a device address):
// the device address of each GPU's copy is looked up once, with that GPU
// current, and kept in scratch_ptr.
static __device__ __align__(256) unsigned char scratch[FLEXATT_NOALLOC_SCRATCH_BYTES];
constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_ptr[kMaxDevices] = {};

// Device address of the scratch copy of the GPU that `stream` runs on, which
// must be the current device (the lookup needs it current).
int scratch_for_stream(hipStream_t stream, void** out) {
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return (int)e;
  if (stream) {
    int sdev = -1;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess) return (int)e;
    if (sdev != cur) return FLEXATT_EINVAL;
  }
  if (cur < 0 || cur >= kMaxDevices) return FLEXATT_EINVAL;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_ptr[cur]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!ptr) return (int)hipErrorInvalidSymbol;
    scratch_ptr[cur] = ptr;
  }
  *out = scratch_ptr[cur];
  return FLEXATT_OK;
}

// Interval and block masks take the general dQ kernel (the recomputing
// D = 128 tile stream has neither); the D = 128 dK/dV tile stream has both.
bool has_masks(const flexatt_problem* p) { return p->doc_bounds || p->block_map; }
BwdLauncher pick_dq(const flexatt_problem* p) {
  // the query-stationary tile stream (bwd_q.hip) has no document, prefix or
  // block-map masks: with them the general kernel runs
  if (has_masks(p) && p->dtype != FLEXATT_F32) {
    const bool bf = p->dtype == FLEXATT_BF16;
    if (p->head_dim == 128) return bf ? bwd_dq_mfma_bf16_d128 : bwd_dq_mfma_f16_d128;
    if (p->head_dim == 64) return bf ? bwd_dq_mfma_bf16_d64 : bwd_dq_mfma_f16_d64;
  }
  return kDq[p->dtype][head_index(p->head_dim)];
}
// The dQ kernel that can also form Delta itself (the D = 64 and 128 tile stream).
bool dq_fuses_delta(const flexatt_problem* p) {
  const BwdLauncher f = pick_dq(p);
  return f == bwd_q_bf16_d128 || f == bwd_q_f16_d128 || f == bwd_q_bf16_d64 || f == bwd_q_f16_d64;
}
BwdLauncher pick_dkdv(const flexatt_problem* p) { return kDkdv[p->dtype][head_index(p->head_dim)]; }

#define FLEXATT_TRY(x)             \
  do {                             \
    const int rc_ = (x);           \
    if (rc_ != FLEXATT_OK) return rc_; \
  } while (0)

// CUs of the current device (cached per device), 0 if unknown.  Host threads
// may call the ABI concurrently: the cache is atomic (a racing first lookup
// stores the same value twice).
int cu_count() {
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

int bwd_common(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k,
               const flexatt_tensor* v, const flexatt_tensor* dout, const float* lse, const float* delta,
               BwdArgs& a) {
  FLEXATT_TRY(check_problem(p));
  FLEXATT_TRY(check_tensor(q, p->dtype));
  FLEXATT_TRY(check_tensor(k, p->dtype));
  FLEXATT_TRY(check_tensor(v, p->dtype));
  FLEXATT_TRY(check_tensor(dout, p->dtype));
  if (!lse || !delta) return FLEXATT_EINVAL;
  a.q = view(q);
  a.k = view(k);
  a.v = view(v);
  a.dout = view(dout);
  a.lse = lse;
  a.delta = delta;
  a.p = make_shape(p);
  a.ntiles = 0;
  a.o = View{nullptr, 0, 0, 0};
  a.delta_out = nullptr;
  a.ds = nullptr;
  a.ds_head = 0;
  a.queue = nullptr;
  a.nstatic = cu_count() & ~7;  // the first round of workgroups (also sets the dK/dV walk direction)
  return FLEXATT_OK;
}

// Staged dS (fp16/bf16 at D = 64, 128 and 256; fp32 at every D;
// every mask primitive: the dK/dV kernel masks per element and stores every
// unit of the causal / window band, zero where masked): units per query head
// and workspace bytes; 0 when the problem takes the recomputing dQ kernel.
bool ds_applies(const flexatt_problem* p) {
  if (p->dtype == FLEXATT_F32) return true;
  return (p->dtype == FLEXATT_F16 || p->dtype == FLEXATT_BF16) &&
         (p->head_dim == 64 || p->head_dim == 128 || p->head_dim == 256);
}
int64_t ds_unit_bytes(const flexatt_problem* p) { return p->dtype == FLEXATT_F32 ? kDsUnitB32 : kDsUnitB; }
BwdLauncher pick_kv_ds(const flexatt_problem* p) {
  if (p->dtype == FLEXATT_F32)
    return p->head_dim == 32 ? bwd_kv_ds_f32_d32
           : p->head_dim == 64 ? bwd_kv_ds_f32_d64
           : p->head_dim == 128 ? bwd_kv_ds_f32_d128 : bwd_kv_ds_f32_d256;
  const bool bf = p->dtype == FLEXATT_BF16;
  if (p->head_dim == 64) return bf ? bwd_kv_ds_bf16_d64 : bwd_kv_ds_f16_d64;
  if (p->head_dim == 256) return bf ? bwd_kv_ds_bf16_d256 : bwd_kv_ds_f16_d256;
  return bf ? bwd_kv_ds_bf16_d128 : bwd_kv_ds_f16_d128;
}
BwdLauncher pick_dq_ds(const flexatt_problem* p) {
  if (p->dtype == FLEXATT_F32)
    return p->head_dim == 32 ? bwd_dq_ds_f32_d32
           : p->head_dim == 64 ? bwd_dq_ds_f32_d64
           : p->head_dim == 128 ? bwd_dq_ds_f32_d128 : bwd_dq_ds_f32_d256;
  const bool bf = p->dtype == FLEXATT_BF16;
  if (p->head_dim == 64) return bf ? bwd_dq_ds_bf16_d64 : bwd_dq_ds_f16_d64;
  if (p->head_dim == 256) return bf ? bwd_dq_ds_bf16_d256 : bwd_dq_ds_f16_d256;
  return bf ? bwd_dq_ds_bf16_d128 : bwd_dq_ds_f16_d128;
}
int64_t ds_units_per_head(const flexatt_problem* p) {
  const int nqt = (p->seqlen_q + kDsQT - 1) / kDsQT;
  const int nkb = (p->seqlen_kv + kDsKB - 1) / kDsKB;
  return ds_tile_offset(nqt, p->causal, p->sliding_window, nkb);
}
size_t ds_bytes(const flexatt_problem* p) {
  if (!ds_applies(p)) return 0;
  return (size_t)((int64_t)p->batch * p->heads_q * ds_units_per_head(p) * ds_unit_bytes(p));
}
int ds_workspace(const flexatt_problem* p, void* ws, size_t bytes, BwdArgs& a) {
  if (!ds_applies(p)) return FLEXATT_ERANGE;
  if (!ws) return FLEXATT_EINVAL;
  if (bytes < ds_bytes(p)) return FLEXATT_EINVAL;
  if (((uintptr_t)ws) % 16 != 0) return FLEXATT_ELAYOUT;
  a.ds = (char*)ws;
  a.ds_head = ds_units_per_head(p);
  return FLEXATT_OK;
}

// Bounded workspaces: the staged backward of a problem whose whole dS band
// exceeds the caller's workspace runs in passes over chunks of (batch, KV
// head) groups, each pass a problem of its own over the same buffers.  A
// group (one KV head and its G query heads) is the smallest chunk: its dK /
// dV sum and its dQ rows need only its own dS units.
int64_t ds_group_bytes(const flexatt_problem* p) {
  return (int64_t)(p->heads_q / p->heads_kv) * ds_units_per_head(p) * ds_unit_bytes(p);
}
// Groups per pass for a workspace of `bytes` (>= one group's band): whole
// batches when at least one batch fits, else KV heads of one batch.
int64_t chunk_groups(const flexatt_problem* p, size_t bytes) {
  int64_t k = (int64_t)(bytes / (size_t)ds_group_bytes(p));
  if (k >= p->heads_kv) k = k / p->heads_kv * p->heads_kv;
  return k;
}
// One pass: batches [b0, b0 + nb) with every KV head, or (nb = 1) the KV
// heads [h0, h0 + nh) of batch b0.
struct Chunk {
  int b0, nb, h0, nh;
};
flexatt_problem sub_problem(const flexatt_problem* p, const Chunk& c) {
  flexatt_problem s = *p;
  const int G = p->heads_q / p->heads_kv;
  s.batch = c.nb;
  s.heads_kv = c.nh;
  s.heads_q = c.nh * G;
  if (p->alibi_slopes) s.alibi_slopes = p->alibi_slopes + (int64_t)c.h0 * G;
  if (p->doc_bounds) s.doc_bounds = p->doc_bounds + (int64_t)c.b0 * p->seqlen_q * 2;
  if (p->col_bounds) s.col_bounds = p->col_bounds + (int64_t)c.b0 * p->seqlen_kv * 2;
  if (p->block_map) {
    const int64_t nq = (p->seqlen_q + kBlk - 1) / kBlk, nk = (p->seqlen_kv + kBlk - 1) / kBlk;
    const bool per_head = p->block_heads == p->heads_q && p->heads_q > 1;
    s.block_map = p->block_map + ((int64_t)c.b0 * p->block_heads + (per_head ? (int64_t)c.h0 * G : 0)) * nq * nk;
    s.block_heads = per_head ? s.heads_q : 1;
  }
  return s;
}
// The chunk's view of a [B, H, S, D] tensor whose head h0 is at `h0`.
flexatt_tensor sub_tensor(const flexatt_tensor* t, int dt, int64_t b0, int64_t h0) {
  flexatt_tensor s = *t;
  s.data = (char*)t->data + (b0 * t->stride_b + h0 * t->stride_h) * (int64_t)elt_size(dt);
  return s;
}

}  // namespace

extern "C" {

int flexatt_abi_version(void) { return FLEXATT_ABI_VERSION; }

const char* flexatt_status_string(int status) {
  switch (status) {
    case FLEXATT_OK: return "ok";
    case FLEXATT_EINVAL: return "invalid argument (null pointer, non-positive size or bad flag)";
    case FLEXATT_EDTYPE: return "unsupported dtype (expected fp32, fp16 or bf16)";
    case FLEXATT_EHEADDIM: return "unsupported head_dim (expected 32, 64, 128 or 256)";
    case FLEXATT_ESHAPE: return "inconsistent shape (heads_q % heads_kv != 0 or sizes overflow)";
    case FLEXATT_ELAYOUT: return "unsupported layout (innermost stride != 1 or rows not 16-byte aligned)";
    case FLEXATT_ERANGE: return "problem outside the entry point's range";
    case FLEXATT_ESCRATCH: return "problem needs more than the library's fixed scratch buffer (FLEXATT_NOALLOC_SCRATCH_BYTES)";
    default: return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown flexatt status";
  }
}

int flexatt_fwd(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k,
                const flexatt_tensor* v, const flexatt_tensor* o, float* lse, void* stream) {
  FLEXATT_TRY(check_problem(p));
  FLEXATT_TRY(check_tensor(q, p->dtype));
  FLEXATT_TRY(check_tensor(k, p->dtype));
  FLEXATT_TRY(check_tensor(v, p->dtype));
  FLEXATT_TRY(check_out_tensor(o, p->dtype, p->batch, p->heads_q, p->seqlen_q, p->head_dim));
  if (!lse) return FLEXATT_EINVAL;
  FwdArgs a;
  a.q = view(q);
  a.k = view(k);
  a.v = view(v);
  a.o = mview(o);
  a.lse = lse;
  a.p = make_shape(p);
  a.nqt = 0;
  return (int)kFwd[p->dtype][head_index(p->head_dim)](a, (hipStream_t)stream);
}

size_t flexatt_fwd_decode_workspace(const flexatt_problem* p) {
  if (check_problem(p) != FLEXATT_OK || !decode_applies(p)) return 0;
  return decode_plan(p).bytes;
}

int flexatt_fwd_decode(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k,
                       const flexatt_tensor* v, const flexatt_tensor* o, float* lse, void* workspace,
                       size_t workspace_bytes, void* stream) {
  FLEXATT_TRY(check_problem(p));
  FLEXATT_TRY(check_tensor(q, p->dtype));
  FLEXATT_TRY(check_tensor(k, p->dtype));
  FLEXATT_TRY(check_tensor(v, p->dtype));
  FLEXATT_TRY(check_out_tensor(o, p->dtype, p->batch, p->heads_q, p->seqlen_q, p->head_dim));
  if (!lse || !workspace) return FLEXATT_EINVAL;
  if (!decode_applies(p)) return FLEXATT_ERANGE;
  const DecodePlan d = decode_plan(p);
  if (workspace_bytes < d.bytes) return FLEXATT_EINVAL;
  if (((uintptr_t)workspace) % 16 != 0) return FLEXATT_ELAYOUT;
  if (d.ntiles == 0) return FLEXATT_EINVAL;
  return decode_run(p, d, q, k, v, o, lse, workspace, (hipStream_t)stream);
}

int flexatt_fwd_decode_noalloc(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k,
                               const flexatt_tensor* v, const flexatt_tensor* o, float* lse, void* stream) {
  FLEXATT_TRY(check_problem(p));
  FLEXATT_TRY(check_tensor(q, p->dtype));
  FLEXATT_TRY(check_tensor(k, p->dtype));
  FLEXATT_TRY(check_tensor(v, p->dtype));
  FLEXATT_TRY(check_out_tensor(o, p->dtype, p->batch, p->heads_q, p->seqlen_q, p->head_dim));
  if (!lse) return FLEXATT_EINVAL;
  if (!decode_applies(p)) return FLEXATT_ERANGE;
  const DecodePlan d = decode_plan(p);
  if (d.ntiles == 0) return FLEXATT_EINVAL;
  // sizes are checked before anything touches the GPU
  if (d.bytes > (size_t)FLEXATT_NOALLOC_SCRATCH_BYTES) return FLEXATT_ESCRATCH;
  void* ws = nullptr;
  FLEXATT_TRY(scratch_for_stream((hipStream_t)stream, &ws));
  return decode_run(p, d, q, k, v, o, lse, ws, (hipStream_t)stream);
}

namespace {
int run_delta(const flexatt_problem* p, const flexatt_tensor* o, const flexatt_tensor* dout, float* delta,
              int* zero, void* stream) {
  FLEXATT_TRY(check_problem(p));
  FLEXATT_TRY(check_tensor(o, p->dtype));
  FLEXATT_TRY(check_tensor(dout, p->dtype));
  if (!delta) return FLEXATT_EINVAL;
  DeltaArgs a;
  a.o = view(o);
  a.dout = view(dout);
  a.delta = delta;
  a.B = p->batch;
  a.H = p->heads_q;
  a.S = p->seqlen_q;
  a.D = p->head_dim;
  a.zero = zero;
  return (int)bwd_delta(p->dtype, a, (hipStream_t)stream);
}
}  // namespace

int flexatt_bwd_delta(const flexatt_problem* p, const flexatt_tensor* o, const flexatt_tensor* dout,
                      float* delta, void* stream) {
  return run_delta(p, o, dout, delta, nullptr, stream);
}

int flexatt_bwd_dq(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k,
                   const flexatt_tensor* v, const flexatt_tensor* dout, const float* lse,
                   const float* delta, const flexatt_tensor* dq, void* stream) {
  BwdArgs a;
  FLEXATT_TRY(bwd_common(p, q, k, v, dout, lse, delta, a));
  FLEXATT_TRY(check_out_tensor(dq, p->dtype, p->batch, p->heads_q, p->seqlen_q, p->head_dim));
  a.dq = mview(dq);
  return (int)pick_dq(p)(a, (hipStream_t)stream);
}

int flexatt_bwd_dq_delta(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k,
                         const flexatt_tensor* v, const flexatt_tensor* o, const flexatt_tensor* dout,
                         const float* lse, float* delta, const flexatt_tensor* dq, void* stream) {
  BwdArgs a;
  FLEXATT_TRY(bwd_common(p, q, k, v, dout, lse, delta, a));
  FLEXATT_TRY(check_tensor(o, p->dtype));
  FLEXATT_TRY(check_out_tensor(dq, p->dtype, p->batch, p->heads_q, p->seqlen_q, p->head_dim));
  if (!dq_fuses_delta(p)) {  // Delta pass, then dQ
    FLEXATT_TRY(flexatt_bwd_delta(p, o, dout, delta, stream));
    a.dq = mview(dq);
    return (int)pick_dq(p)(a, (hipStream_t)stream);
  }
  a.o = view(o);
  a.delta_out = delta;
  a.dq = mview(dq);
  return (int)pick_dq(p)(a, (hipStream_t)stream);
}

int flexatt_bwd_dkdv(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k,
                     const flexatt_tensor* v, const flexatt_tensor* dout, const float* lse,
                     const float* delta, const flexatt_tensor* dk, const flexatt_tensor* dv,
                     void* stream) {
  BwdArgs a;
  FLEXATT_TRY(bwd_common(p, q, k, v, dout, lse, delta, a));
  FLEXATT_TRY(check_out_tensor(dk, p->dtype, p->batch, p->heads_kv, p->seqlen_kv, p->head_dim));
  FLEXATT_TRY(check_out_tensor(dv, p->dtype, p->batch, p->heads_kv, p->seqlen_kv, p->head_dim));
  a.dk = mview(dk);
  a.dv = mview(dv);
  return (int)pick_dkdv(p)(a, (hipStream_t)stream);
}

int flexatt_bwd(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k,
                const flexatt_tensor* v, const flexatt_tensor* o, const flexatt_tensor* dout,
                const float* lse, float* delta, const flexatt_tensor* dq, const flexatt_tensor* dk,
                const flexatt_tensor* dv, void* stream) {
  BwdArgs a;
  FLEXATT_TRY(bwd_common(p, q, k, v, dout, lse, delta, a));
  FLEXATT_TRY(check_tensor(o, p->dtype));
  FLEXATT_TRY(check_out_tensor(dq, p->dtype, p->batch, p->heads_q, p->seqlen_q, p->head_dim));
  FLEXATT_TRY(check_out_tensor(dk, p->dtype, p->batch, p->heads_kv, p->seqlen_kv, p->head_dim));
  FLEXATT_TRY(check_out_tensor(dv, p->dtype, p->batch, p->heads_kv, p->seqlen_kv, p->head_dim));
  FLEXATT_TRY(flexatt_bwd_dq_delta(p, q, k, v, o, dout, lse, delta, dq, stream));
  a.dk = mview(dk);
  a.dv = mview(dv);
  return (int)pick_dkdv(p)(a, (hipStream_t)stream);
}

size_t flexatt_bwd_workspace(const flexatt_problem* p) {
  if (check_problem(p) != FLEXATT_OK) return 0;
  const size_t n = ds_bytes(p);
  return n ? n + FLEXATT_BWD_QUEUE_BYTES : 0;
}

int flexatt_bwd_prefers_staging(const flexatt_problem* p) {
  if (flexatt_bwd_workspace(p) == 0) return 0;  // outside the staged range (or an invalid problem)
  // fp16/bf16 at head_dim 64 without soft-cap and without document, prefix or
  // block-map masks: the recomputing backward (the query-stationary dQ kernel
  // forming Delta, dK/dV without dS stores) measured 2-15% faster than
  // staging; with soft-cap its tanh recompute in dQ makes it 0-8% slower
  if (p->dtype != FLEXATT_F32 && p->head_dim == 64 && !(p->soft_cap > 0.f) && !has_masks(p)) return 0;
  return 1;
}

size_t flexatt_bwd_workspace_limited(const flexatt_problem* p, size_t limit_bytes) {
  const size_t full = flexatt_bwd_workspace(p);
  if (full == 0 || full <= limit_bytes) return full;
  const size_t gb = (size_t)ds_group_bytes(p);
  if (limit_bytes < gb + FLEXATT_BWD_QUEUE_BYTES) return 0;  // not even one group: recompute
  return (size_t)chunk_groups(p, limit_bytes - FLEXATT_BWD_QUEUE_BYTES) * gb + FLEXATT_BWD_QUEUE_BYTES;
}

namespace {
int run_dkdv_ds(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k, const flexatt_tensor* v,
                const flexatt_tensor* dout, const float* lse, const float* delta, const flexatt_tensor* dk,
                const flexatt_tensor* dv, void* workspace, size_t workspace_bytes, int* queue, void* stream) {
  BwdArgs a;
  FLEXATT_TRY(bwd_common(p, q, k, v, dout, lse, delta, a));
  FLEXATT_TRY(check_out_tensor(dk, p->dtype, p->batch, p->heads_kv, p->seqlen_kv, p->head_dim));
  FLEXATT_TRY(check_out_tensor(dv, p->dtype, p->batch, p->heads_kv, p->seqlen_kv, p->head_dim));
  FLEXATT_TRY(ds_workspace(p, workspace, workspace_bytes, a));
  a.dk = mview(dk);
  a.dv = mview(dv);
  a.queue = queue;
  a.nstatic = cu_count() & ~7;
  return (int)pick_kv_ds(p)(a, (hipStream_t)stream);
}

int run_dq_ds(const flexatt_problem* p, const flexatt_tensor* k, const void* workspace, size_t workspace_bytes,
              const flexatt_tensor* dq, int* queue, void* stream) {
  FLEXATT_TRY(check_problem(p));
  FLEXATT_TRY(check_tensor(k, p->dtype));
  FLEXATT_TRY(check_out_tensor(dq, p->dtype, p->batch, p->heads_q, p->seqlen_q, p->head_dim));
  BwdArgs a;
  a.k = view(k);
  a.dq = mview(dq);
  a.p = make_shape(p);
  a.ntiles = 0;
  a.delta_out = nullptr;
  a.queue = queue;
  a.nstatic = cu_count() & ~7;
  FLEXATT_TRY(ds_workspace(p, (void*)workspace, workspace_bytes, a));
  return (int)pick_dq_ds(p)(a, (hipStream_t)stream);
}
}  // namespace

int flexatt_bwd_dkdv_ds(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k,
                        const flexatt_tensor* v, const flexatt_tensor* dout, const float* lse, const float* delta,
                        const flexatt_tensor* dk, const flexatt_tensor* dv, void* workspace,
                        size_t workspace_bytes, void* stream) {
  return run_dkdv_ds(p, q, k, v, dout, lse, delta, dk, dv, workspace, workspace_bytes, nullptr, stream);
}

int flexatt_bwd_dq_ds(const flexatt_problem* p, const flexatt_tensor* k, const void* workspace,
                      size_t workspace_bytes, const flexatt_tensor* dq, void* stream) {
  return run_dq_ds(p, k, workspace, workspace_bytes, dq, nullptr, stream);
}

namespace {
// One staged pass (the arguments are checked): Delta, dK/dV writing dS, dQ.
int run_staged(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k, const flexatt_tensor* v,
               const flexatt_tensor* o, const flexatt_tensor* dout, const float* lse, float* delta,
               const flexatt_tensor* dq, const flexatt_tensor* dk, const flexatt_tensor* dv, void* workspace,
               size_t workspace_bytes, void* stream) {
  // queue counters after the dS band: [0] the dK/dV launch, [2] dQ
  int* queue = nullptr;
  if (workspace_bytes >= ds_bytes(p) + FLEXATT_BWD_QUEUE_BYTES && (cu_count() & ~7) > 0)
    queue = (int*)((char*)workspace + ds_bytes(p));
  FLEXATT_TRY(run_delta(p, o, dout, delta, queue, stream));
  FLEXATT_TRY(run_dkdv_ds(p, q, k, v, dout, lse, delta, dk, dv, workspace, workspace_bytes, queue, stream));
  return run_dq_ds(p, k, workspace, workspace_bytes, dq, queue ? queue + 2 : nullptr, stream);
}
}  // namespace

int flexatt_bwd_ws(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k,
                   const flexatt_tensor* v, const flexatt_tensor* o, const flexatt_tensor* dout, const float* lse,
                   float* delta, const flexatt_tensor* dq, const flexatt_tensor* dk, const flexatt_tensor* dv,
                   void* workspace, size_t workspace_bytes, void* stream) {
  FLEXATT_TRY(check_problem(p));
  // outside the range, or no workspace at all: the recomputing backward
  if (!ds_applies(p) || (!workspace && workspace_bytes == 0))
    return flexatt_bwd(p, q, k, v, o, dout, lse, delta, dq, dk, dv, stream);
  BwdArgs a;
  FLEXATT_TRY(bwd_common(p, q, k, v, dout, lse, delta, a));
  FLEXATT_TRY(check_tensor(o, p->dtype));
  FLEXATT_TRY(check_out_tensor(dq, p->dtype, p->batch, p->heads_q, p->seqlen_q, p->head_dim));
  FLEXATT_TRY(check_out_tensor(dk, p->dtype, p->batch, p->heads_kv, p->seqlen_kv, p->head_dim));
  FLEXATT_TRY(check_out_tensor(dv, p->dtype, p->batch, p->heads_kv, p->seqlen_kv, p->head_dim));
  if (!workspace) return FLEXATT_EINVAL;
  if (((uintptr_t)workspace) % 16 != 0) return FLEXATT_ELAYOUT;
  if (workspace_bytes >= ds_bytes(p))
    return run_staged(p, q, k, v, o, dout, lse, delta, dq, dk, dv, workspace, workspace_bytes, stream);
  // A smaller workspace: passes over chunks of whole (batch, KV head) groups.
  if (workspace_bytes < (size_t)ds_group_bytes(p)) return FLEXATT_EINVAL;
  const int64_t kg = chunk_groups(p, workspace_bytes);
  const int G = p->heads_q / p->heads_kv;
  const int nbc = kg >= p->heads_kv ? (int)(kg / p->heads_kv) : 1;  // batches per pass
  const int nhc = kg >= p->heads_kv ? p->heads_kv : (int)kg;        // KV heads per pass
  for (int b0 = 0; b0 < p->batch; b0 += nbc)
    for (int h0 = 0; h0 < p->heads_kv; h0 += nhc) {
      const Chunk c{b0, nbc < p->batch - b0 ? nbc : p->batch - b0, h0, nhc < p->heads_kv - h0 ? nhc : p->heads_kv - h0};
      const flexatt_problem sp = sub_problem(p, c);
      const int64_t hq0 = (int64_t)h0 * G;
      const flexatt_tensor sq = sub_tensor(q, p->dtype, b0, hq0), sk = sub_tensor(k, p->dtype, b0, h0),
                           sv = sub_tensor(v, p->dtype, b0, h0), so = sub_tensor(o, p->dtype, b0, hq0),
                           sdo = sub_tensor(dout, p->dtype, b0, hq0), sdq = sub_tensor(dq, p->dtype, b0, hq0),
                           sdk = sub_tensor(dk, p->dtype, b0, h0), sdv = sub_tensor(dv, p->dtype, b0, h0);
      const int64_t r0 = ((int64_t)b0 * p->heads_q + hq0) * p->seqlen_q;  // first LSE / Delta row
      FLEXATT_TRY(run_staged(&sp, &sq, &sk, &sv, &so, &sdo, lse + r0, delta + r0, &sdq, &sdk, &sdv, workspace,
                             workspace_bytes, stream));
    }
  return FLEXATT_OK;
}

}  // extern "C"
