// fp32 flash-attention dQ on the vector ALUs, recomputing S and dP.
//
// The library's fp32 path runs on the fp32 matrix cores (f32_mfma.hip); this
// kernel serves the one fp32 case left: the dQ of the backward without a dS
// workspace (flexatt_bwd, flexatt_bwd_dq) at head_dim 256, whose Q, dO and dQ
// rows (768 values per lane for a 32-row block) exceed one lane's registers
// on the matrix cores.  The reference accepts fp32 tensors on the same entry
// points (test/test_supplementary.py:55-63; the fp32 suites of
// test/test_comprehensive.py) and expects fp32-exact results (tolerances down
// to 1e-5, test/test_comprehensive.py:88): one 16-lane group per row, K/V
// tiles staged in LDS, fp32 FMA, softmax terms in the natural domain with
// expf/tanhf.  Semantics are those of the MFMA kernels
// (npu_flash_attention.py:298-402), including the KV tail and ALiBi.
#include "flexatt_device.h"
#include "flexatt_kernels.h"

#ifndef FLEXATT_D
#error "FLEXATT_D (head dim) must be defined"
#endif

namespace flexatt {

namespace simt {
constexpr int kRows = 16;   // rows per workgroup (one 16-lane group each)
constexpr int kLanes = 16;  // lanes per row
constexpr int kTile = 32;   // rows per LDS tile

__device__ __forceinline__ float group_sum(float x) {
  x += __shfl_xor(x, 8);
  x += __shfl_xor(x, 4);
  x += __shfl_xor(x, 2);
  x += __shfl_xor(x, 1);
  return x;
}

// Natural-domain transformed score; t receives tanh(scale*s/cap).
__device__ __forceinline__ float score(float s, const Shape& p, float slope, int i, int j, float& t) {
  float x = s * p.scale;
  if (p.cap > 0.f) {
    t = tanhf(x * p.inv_cap);
    x = p.cap * t;
  }
  if (p.alibi) x += slope * (float)(i - j);
  return x;
}
}  // namespace simt

template <int D>
__global__ __launch_bounds__(256) void bwd_dq_simt_kernel(BwdArgs a) {
  using namespace simt;
  constexpr int E = D / kLanes;
  __shared__ float sK[kTile][D];
  __shared__ float sV[kTile][D];
  const Shape& p = a.p;
  const int tid = threadIdx.x, rg = tid / kLanes, ln = tid % kLanes;
  const int qt = blockIdx.x % a.ntiles, bh = blockIdx.x / a.ntiles;
  const int hq = bh % p.Hq, b = bh / p.Hq, hk = hq / p.G;
  const int m0 = qt * kRows, my_m = m0 + rg;
  const float* qp = (const float*)a.q.data + b * a.q.sb + hq * a.q.sh;
  const float* dop = (const float*)a.dout.data + b * a.dout.sb + hq * a.dout.sh;
  const float* kp = (const float*)a.k.data + b * a.k.sb + hk * a.k.sh;
  const float* vp = (const float*)a.v.data + b * a.v.sb + hk * a.v.sh;
  float q[E], dO[E], dq[E];
  const int rq = min(my_m, p.Sq - 1);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    q[e] = my_m < p.Sq ? qp[(int64_t)rq * a.q.ss + ln + kLanes * e] : 0.f;
    dO[e] = my_m < p.Sq ? dop[(int64_t)rq * a.dout.ss + ln + kLanes * e] : 0.f;
    dq[e] = 0.f;
  }
  float lse = kPosInf, dl = 0.f;
  if (my_m < p.Sq) {
    const int64_t ri = (int64_t)(b * p.Hq + hq) * p.Sq + my_m;
    lse = a.lse[ri] == kNegInf ? kPosInf : a.lse[ri];
    dl = a.delta[ri];
  }
  const float slope = p.alibi ? p.alibi[hq] : 0.f;
  int kv_lo = 0, kv_hi = p.Skv;
  if (p.causal) kv_hi = min(kv_hi, m0 + kRows);
  if (p.window > 0) kv_lo = max(0, m0 - p.window);
  int dlo, dhi;
  doc_bounds(p, b, rq, dlo, dhi);
  if (p.doc) {  // KV range of the block's documents
    int l0, h0, l1, h1;
    doc_bounds(p, b, min(m0, p.Sq - 1), l0, h0);
    doc_bounds(p, b, min(m0 + kRows, p.Sq) - 1, l1, h1);
    kv_lo = max(kv_lo, l0);
    kv_hi = min(kv_hi, h1);
  }
  for (int n0 = (kv_lo / kTile) * kTile; n0 < kv_hi; n0 += kTile) {
    __syncthreads();
    for (int idx = tid; idx < kTile * D; idx += 256) {
      const int r = idx / D, c = idx % D, n = n0 + r;
      const int nc = min(n, p.Skv - 1);
      sK[r][c] = n < p.Skv ? kp[(int64_t)nc * a.k.ss + c] : 0.f;
      sV[r][c] = n < p.Skv ? vp[(int64_t)nc * a.v.ss + c] : 0.f;
    }
    __syncthreads();
#pragma unroll 4
    for (int jj = 0; jj < kTile; ++jj) {
      float s = 0.f, dpv = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        s = fmaf(q[e], sK[jj][ln + kLanes * e], s);
        dpv = fmaf(dO[e], sV[jj][ln + kLanes * e], dpv);
      }
      s = group_sum(s);
      dpv = group_sum(dpv);
      const int j = n0 + jj;
      float t = 0.f;
      const float x = score(s, p, slope, my_m, j, t);
      const float pj = (allowed(p, my_m, j) && j >= dlo && j < dhi && block_on(p, b, hq, min(my_m, p.Sq - 1), j))
                           ? expf(x - lse)
                           : 0.f;
      float ds = pj * (dpv - dl) * p.scale;
      if (p.cap > 0.f) ds *= (1.0f - t * t);
#pragma unroll
      for (int e = 0; e < E; ++e) dq[e] = fmaf(ds, sK[jj][ln + kLanes * e], dq[e]);
    }
  }
  if (my_m < p.Sq) {
    float* op = (float*)a.dq.data + b * a.dq.sb + hq * a.dq.sh + (int64_t)my_m * a.dq.ss;
#pragma unroll
    for (int e = 0; e < E; ++e) op[ln + kLanes * e] = dq[e];
  }
}

#define FLEXATT_CAT2(a, b) a##b
#define FLEXATT_CAT(a, b) FLEXATT_CAT2(a, b)
#if FLEXATT_D == 256
hipError_t FLEXATT_CAT(bwd_dq_simt_f32_d, FLEXATT_D)(const BwdArgs& a, hipStream_t st) {
  BwdArgs x = a;
  x.ntiles = (a.p.Sq + simt::kRows - 1) / simt::kRows;
  hipLaunchKernelGGL((bwd_dq_simt_kernel<FLEXATT_D>), dim3(x.ntiles * a.p.B * a.p.Hq), dim3(256), 0, st, x);
  return hipGetLastError();
}

#endif

}  // namespace flexatt
