// Split-KV forward for few query rows per KV head (flash-decoding): KV-cache
// decoding, where Sq is tiny and Skv long, so that the regular forward's one
// workgroup per (batch, KV head, query tile) leaves most of the GPU idle and
// pads every query row to a 32-row MFMA tile per head.
//
// Semantics: those of the forward, npu_flash_attention.py:17-166 (score order
// scale -> soft-cap -> ALiBi -> mask, online softmax in the log2 domain, LSE
// in natural log).  The reference sketches the same split at :169-293
// (flash_attn_fwd_split_kv_kernel / flash_attn_fwd_reduce_kernel) but never
// calls it; this is a gfx950 design of its own.
//
// Decomposition
//  * All G = Hq / Hkv heads of a KV head and all Sq query rows are packed
//    into the 32 columns of one MFMA tile: column r = g * Sq + i for head
//    hk * G + g and query row i (G * Sq <= 32; unused columns repeat the last
//    row and are not written).  K and V are read once for all of them.
//  * One workgroup = 4 waves for one (b, hkv) and one contiguous chunk of
//    32-row KV tiles; wave w takes tiles w, w + 4, ... of the chunk on its
//    own: its own LDS stages (K with the column-read swizzle, V with the
//    transpose-read swizzle, direct-to-LDS copies one tile ahead), its own
//    online softmax, no barriers.
//  * The waves' online-softmax states are combined through LDS into one
//    partial result per workgroup: O normalised by its row sums (fp32) and
//    its LSE in log2 units, in the caller's workspace.  A merge kernel (one
//    thread per output element) combines the partials of a row in a fixed
//    order: M = max LSE_s, O = sum 2^(LSE_s - M) O_s / sum 2^(LSE_s - M),
//    LSE = (M + log2 sum 2^(LSE_s - M)) ln 2.  Deterministic.
#include "flexatt_device.h"
#include "flexatt_kernels.h"

#ifndef FLEXATT_D
#error "FLEXATT_D (head dim) must be defined"
#endif

namespace flexatt {

#if FLEXATT_D <= 128

constexpr float kDecRescale = 8.0f;  // lazy rescale threshold, log2 units (as the forward)

template <int D>
struct DecCfg {
  static constexpr int NW = 4;  // waves per workgroup
  static constexpr int BN = 32;          // KV rows per tile
  static constexpr int KC = D / 16;      // k steps of S^T = K Q^T
  static constexpr int DB = D / 32;      // 32-row blocks of O^T
  static constexpr int CPR = D / 8;      // 16-byte chunks per row
  static constexpr int ROWB = 2 * D;     // bytes per row
  static constexpr int TB = BN * ROWB;   // bytes of one K or V tile
  static constexpr int E = TB / 1024;    // 1 KB copies per tile per tensor
  // tiles in LDS per wave, STAGES - 1 in flight.  Measured: four waves with
  // two stages beat two (D = 128) or four waves with four stages (fewer
  // waves per CU), 5.6 against 4.6 TB/s at D = 128.
  static constexpr int STAGES = 2;
  static constexpr int WAVEB = STAGES * 2 * TB;  // LDS bytes per wave
  static_assert(E >= 1 && E * 1024 == TB, "tile must split into 1 KB copies");
};

template <class T, int D, bool SOFTCAP, bool ALIBI>
__global__ __launch_bounds__(DecCfg<D>::NW * 64) void fwd_decode_kernel(DecodeArgs a) {
  using C = DecCfg<D>;
  using M = Mfma<T>;
  using V8 = typename M::v8;
  __shared__ __attribute__((aligned(1024))) char smem[C::NW * C::WAVEB];

  const Shape& p = a.p;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31;

  // Work item: (b, hkv, split); splits of one (b, hkv) are consecutive.
  const int s = blockIdx.x % a.nsplit;
  const int bh = blockIdx.x / a.nsplit;
  const int hk = bh % p.Hkv, b = bh / p.Hkv;

  // Packed query column of this lane.
  const int R = p.G * p.Sq;
  const int r = min(l32, R - 1);
  const int g = r / p.Sq, qi = r % p.Sq;
  const int hq = hk * p.G + g;

  // Q^T as MFMA B operands (k = 8 consecutive d of query row qi).
  V8 qf[C::KC];
  {
    const T* src = (const T*)a.q.data + b * a.q.sb + hq * a.q.sh + (int64_t)qi * a.q.ss + 8 * h;
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc) qf[kc] = as_v8<V8>(ld_global16(src + 16 * kc));
  }
  constexpr bool RAW = !SOFTCAP && !ALIBI;
  float c2 = p.scale_log2;
  if constexpr (RAW) {  // as in the forward: a negative scale moves into Q
    if (c2 < 0.f) {
#pragma unroll
      for (int kc = 0; kc < C::KC; ++kc)
        qf[kc] = as_v8<V8>(__builtin_bit_cast(i32x4, qf[kc]) ^ i32x4{(int)0x80008000, (int)0x80008000,
                                                                     (int)0x80008000, (int)0x80008000});
      c2 = -c2;
    }
    if (c2 == 0.f) c2 = 1e-30f;
  }
  const float slope_log2 = ALIBI ? p.alibi[hq] * kLog2e : 0.f;

  // This wave's tiles: t = c_lo + wave + NW * j, t < c_hi.
  const int c_lo = s * a.chunk;
  const int c_hi = min(c_lo + a.chunk, a.ntiles);
  const int first = c_lo + wave;
  const int nt = first < c_hi ? (c_hi - first + C::NW - 1) / C::NW : 0;

  const T* kp = (const T*)a.k.data + b * a.k.sb + hk * a.k.sh;
  const T* vp = (const T*)a.v.data + b * a.v.sb + hk * a.v.sh;
  const unsigned wbase = lds_addr_of(smem) + wave * C::WAVEB;
  auto issue = [&](int t, int st) {
    const int n0 = t * C::BN;
    const unsigned sb = wbase + st * 2 * C::TB;
#pragma unroll
    for (int e = 0; e < C::E; ++e) {
      const int q = e * 64 + lane;
      const int row = q / C::CPR, pc = q % C::CPR;
      const int64_t n = min(n0 + row, p.Skv - 1);
      load_lds16(kp + n * a.k.ss + swz_col<C::CPR>(row, pc) * 8, sb + e * 1024);
      load_lds16(vp + n * a.v.ss + swz_tr_inv<C::CPR>(row, pc) * 8, sb + C::TB + e * 1024);
    }
  };

  int koff[C::KC], voff[C::DB];
  {
    const int tr_row = 4 * h + ((lane & 15) >> 2);
    const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc) koff[kc] = l32 * C::ROWB + swz_col<C::CPR>(l32, 2 * kc + h) * 16;
#pragma unroll
    for (int db = 0; db < C::DB; ++db)
      voff[db] = tr_row * C::ROWB + swz_tr<C::CPR>(tr_row, 4 * db + (tr_col >> 3)) * 16 + (tr_col & 7) * 2;
  }

  f32x16 acc[C::DB];
#pragma unroll
  for (int db = 0; db < C::DB; ++db) acc[db] = f32x16{};
  float m_run = kNegInf, l_run = 0.f;

  // Tiles STAGES - 1 ahead: the copy of tile j + STAGES - 1 goes to the stage
  // of tile j - 1, read in the previous iteration.  Near the end (nothing left
  // to issue) the wait drains every copy.
#pragma unroll
  for (int j = 0; j < C::STAGES - 1; ++j)
    if (j < nt) issue(first + C::NW * j, j);
  for (int j = 0; j < nt; ++j) {
    const int t = first + C::NW * j;
    if (j + C::STAGES - 1 < nt) {
      issue(t + C::NW * (C::STAGES - 1), (j + C::STAGES - 1) % C::STAGES);
      wait_vmcnt<(C::STAGES - 1) * 2 * C::E>();  // tile t landed, the next STAGES - 1 in flight
    } else {
      wait_vmcnt<0>();
    }
    const char* sK = smem + wave * C::WAVEB + (j % C::STAGES) * 2 * C::TB;
    const char* sV = sK + C::TB;
    const int n0 = t * C::BN;

    f32x16 sc = f32x16{};
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc) sc = M::mma(as_v8<V8>(lds_read16(sK + koff[kc])), qf[kc], sc);

    // element e is KV row n0 + 8(e/4) + 4h + e%4, query row qi of head hq
    if constexpr (!RAW) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int jj = n0 + 8 * (e >> 2) + 4 * h + (e & 3);
        float tv;
        sc[e] = score_log2<SOFTCAP, ALIBI>(sc[e], p, slope_log2, qi, jj, tv);
      }
    }
    const bool need_mask = (n0 + C::BN > p.Skv) || p.causal || (p.window > 0 && (p.Sq - 1) - n0 > p.window);
    if (need_mask) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int jj = n0 + 8 * (e >> 2) + 4 * h + (e & 3);
        if (!allowed(p, qi, jj)) sc[e] = kNegInf;
      }
    }
    float mx, mx2;
    max16_partial(sc, mx, mx2);
    mx = max2(mx, mx2);
    if constexpr (RAW) mx *= c2;
    mx = fmaxf(mx, swap_halves(mx));
    if (mx != mx) mx = kNegInf;
    const bool grow = mx > m_run + kDecRescale;
    if (__builtin_amdgcn_ballot_w64(grow)) {
      const float m_new = grow ? mx : m_run;
      const float alpha = grow ? fast_exp2(m_run - m_new) : 1.f;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < C::DB; ++db) scale_inplace(acc[db], alpha);
      m_run = m_new;
    }
    const float m_use = (m_run == kNegInf) ? 0.f : m_run;
    f32x16 pe;
    float rs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      if constexpr (RAW) pe[e] = fast_exp2(__builtin_fmaf(sc[e], c2, -m_use));
      else pe[e] = fast_exp2(sc[e] - m_use);
      rs[e & 3] += pe[e];
    }
    l_run += (rs[0] + rs[1]) + (rs[2] + rs[3]);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const V8 pb = pack8<T>(pe, 8 * c);
      const char* vr = sV + 16 * c * C::ROWB;
#pragma unroll
      for (int db = 0; db < C::DB; ++db) {
        const i16x4 lo = lds_read_tr4(vr + voff[db]);
        const i16x4 hi = lds_read_tr4(vr + 8 * C::ROWB + voff[db]);
        acc[db] = M::mma(cat_tr<V8>(lo, hi), pb, acc[db]);
      }
    }
  }

  // The workgroup's partial result: the NW waves' (m, l, acc) combined in a
  // fixed order through LDS (every wave's copies have landed: its last tile
  // waited for vmcnt 0), then O / l (fp32) and LSE in log2 units.
  const float l_tot = l_run + swap_halves(l_run);  // this wave's row sum
  __syncthreads();
  float* xm = (float*)smem;         // [NW][64]
  float* xl = xm + C::NW * 64;      // [NW][64]
  float* xa = xl + C::NW * 64;      // [NW][DB][16][64]
  xm[wave * 64 + lane] = m_run;
  xl[wave * 64 + lane] = l_tot;
#pragma unroll
  for (int db = 0; db < C::DB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) xa[((wave * C::DB + db) * 16 + e) * 64 + lane] = acc[db][e];
  __syncthreads();
  float mw[C::NW], mall = kNegInf;
#pragma unroll
  for (int w = 0; w < C::NW; ++w) {
    mw[w] = xm[w * 64 + lane];
    mall = fmaxf(mall, mw[w]);
  }
  float al[C::NW], L = 0.f;
#pragma unroll
  for (int w = 0; w < C::NW; ++w) {
    al[w] = mw[w] == kNegInf ? 0.f : fast_exp2(mw[w] - mall);  // 0 for a wave without keys
    L = __builtin_fmaf(al[w], xl[w * 64 + lane], L);
  }
  const bool empty = !(L > 0.f);
  const float inv = empty ? 0.f : 1.0f / L;
  if (l32 < R) {
    const int64_t row = ((int64_t)b * p.Hq + hq) * p.Sq + qi;
    float* po = a.part_o + (row * a.nsplit + s) * D + 4 * h;
    for (int db = wave; db < C::DB; db += C::NW) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < C::NW; ++w)
#pragma unroll
          for (int j = 0; j < 4; ++j) o[j] = __builtin_fmaf(al[w], xa[((w * C::DB + db) * 16 + 4 * i + j) * 64 + lane], o[j]);
        *(f32x4*)(po + 32 * db + 8 * i) = o * inv;
      }
    }
    if (wave == 0 && h == 0) a.part_lse[row * a.nsplit + s] = empty ? kNegInf : mall + log2f(L);
  }
}

// Merge of the workgroups' partials: one thread per output element, the
// partials of its row in order.
template <class T, int D>
__global__ __launch_bounds__(256) void fwd_decode_merge_kernel(DecodeArgs a) {
  const Shape& p = a.p;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t rows = (int64_t)p.B * p.Hq * p.Sq;
  if (gid >= rows * D) return;
  const int64_t row = gid / D;
  const int d = (int)(gid % D);
  const int ns = a.nsplit;
  const float* pl = a.part_lse + row * ns;
  float mx = kNegInf;
  for (int s = 0; s < ns; ++s) mx = fmaxf(mx, pl[s]);
  const int i = (int)(row % p.Sq);
  const int64_t bh = row / p.Sq;
  const int hq = (int)(bh % p.Hq), b = (int)(bh / p.Hq);
  T* out = (T*)a.o.data + b * a.o.sb + hq * a.o.sh + (int64_t)i * a.o.ss;
  if (mx == kNegInf) {  // no allowed key for this row
    out[d] = from_f32<T>(0.f);
    if (d == 0) a.lse[row] = kNegInf;
    return;
  }
  const float* po = a.part_o + row * ns * D + d;
  float ws = 0.f, acc = 0.f;
#pragma unroll 8
  for (int s = 0; s < ns; ++s) {
    const float w = fast_exp2(pl[s] - mx);  // 0 for an empty partial
    ws += w;
    acc = __builtin_fmaf(w, po[(int64_t)s * D], acc);
  }
  out[d] = from_f32<T>(acc / ws);
  if (d == 0) a.lse[row] = (mx + log2f(ws)) * kLn2;
}

template <class T, int D>
hipError_t launch_decode(const DecodeArgs& a, hipStream_t st) {
  using C = DecCfg<D>;
  const dim3 grid(a.nsplit * a.p.B * a.p.Hkv), block(C::NW * 64);
  const bool sc = a.p.cap > 0.f, al = a.p.alibi != nullptr;
  if (sc && al) hipLaunchKernelGGL((fwd_decode_kernel<T, D, true, true>), grid, block, 0, st, a);
  else if (sc) hipLaunchKernelGGL((fwd_decode_kernel<T, D, true, false>), grid, block, 0, st, a);
  else if (al) hipLaunchKernelGGL((fwd_decode_kernel<T, D, false, true>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((fwd_decode_kernel<T, D, false, false>), grid, block, 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t n = (int64_t)a.p.B * a.p.Hq * a.p.Sq * D;
  hipLaunchKernelGGL((fwd_decode_merge_kernel<T, D>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a);
  return hipGetLastError();
}

#define FLEXATT_CAT2(a, b) a##b
#define FLEXATT_CAT(a, b) FLEXATT_CAT2(a, b)
hipError_t FLEXATT_CAT(fwd_decode_bf16_d, FLEXATT_D)(const DecodeArgs& a, hipStream_t st) {
  return launch_decode<__bf16, FLEXATT_D>(a, st);
}
hipError_t FLEXATT_CAT(fwd_decode_f16_d, FLEXATT_D)(const DecodeArgs& a, hipStream_t st) {
  return launch_decode<_Float16, FLEXATT_D>(a, st);
}

#endif  // FLEXATT_D <= 128

}  // namespace flexatt
