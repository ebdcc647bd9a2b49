// fp32 flash attention on the fp32 matrix cores: forward, dQ (from the
// staged dS, or recomputing S and dP) and dK/dV for fp32 inputs.
//
// The reference accepts fp32 tensors on the same entry points
// (test/test_supplementary.py:55-63; the fp32 suites of
// test/test_comprehensive.py) and expects fp32-exact results (tolerances down
// to 1e-5, test/test_comprehensive.py:88).  These kernels multiply in fp32 on
// the matrix cores (each product and sum rounded to fp32, as an fp32 FMA
// chain is) and keep the softmax in the natural domain with expf/logf/tanhf,
// as the reference's fp32 math does (npu_flash_attention.py:17-166, :298-402,
// :407-560).  Semantics are those of the 16-bit kernels: KV tail, causal,
// sliding window, soft-cap, ALiBi, interval and block masks, and the GQA
// group sum inside dK/dV.
//
// Two MFMA shapes, one operand value per lane per instruction:
//  * v_mfma_f32_32x32x2_f32 (the forward and the dQ from the staged dS):
//      A operand  lane l holds A[row = l%32][k = l/32]
//      B operand  lane l holds B[k = l/32][col = l%32]
//      C/D        acc[4*i + j] = C[row = 8*i + 4*(l/32) + j][col = l%32]
//    A product over the head dim runs as D/2 MFMAs; wave half h takes
//    d = h*D/2 + s at step s, so that each lane reads its operand rows as
//    contiguous 16-byte groups.  A product over 32 rows (P V, dS K) takes at
//    step r the rows 8*(r/4) + 4h + r%4 -- exactly the rows whose scores
//    lane half h holds in accumulator element r, so the scores feed the B
//    operand from their own registers.
//  * v_mfma_f32_16x16x4_f32 (dK/dV and the recomputing dQ, 16 rows per
//    wave, half the per-lane state): layout and step order given with it
//    below.
//
// Forward and dQ keep the query rows as the accumulator columns
// (S^T = K Q^T, one query row per lane); dK/dV keeps the KV rows as columns
// (S = Q K^T, one KV row per lane).  K/V (or Q/dO) tiles of 32 rows pass
// through registers (at D = 256: one direct-to-LDS load per row) into a
// double-buffered LDS tile with rows padded to D + 4 floats (16-byte row
// reads and 4-byte column reads both without bank conflicts), one barrier
// per tile.
#include "flexatt_device.h"
#include "flexatt_kernels.h"

#ifndef FLEXATT_D
#error "FLEXATT_D (head dim) must be defined"
#endif

namespace flexatt {

namespace f32m {

constexpr int kTile = 32;  // rows per LDS tile (one MFMA block)

__device__ __forceinline__ f32x16 mma(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Row of the 32-row block that lane half h takes at step r (and that holds
// accumulator element r).
__device__ __forceinline__ int blk_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

template <int D, int NW>
struct Cfg {
  static constexpr int NT = NW * 64;              // threads per workgroup
  static constexpr int P = D + 4;                 // LDS row pitch (floats)
  static constexpr int TILE = kTile * P;          // floats per LDS tile
  static constexpr int N4 = kTile * D / 4;        // 16-byte pieces per tile
  static constexpr int NL = (N4 + NT - 1) / NT;   // pieces per thread per tensor
  static constexpr int HD = D / 2;                // head-dim values per lane for the d-sums
  static constexpr int DB = D / 32;               // 32-wide head-dim blocks
};

// One 32-row tile of one tensor into an LDS tile of D + 4-float rows.
// fetch() starts the copy, commit() completes it in the issuing thread,
// settle() (before the barrier that publishes the tile) waits for it.  At
// D = 256 a row is 1 KB, one direct-to-LDS load of the wave (lane l's 16
// bytes at row offset 16 l), so the copy holds no registers.  Otherwise the
// copy passes through registers, which nothing reads before commit() (so
// the loads overlap the work between the two calls).  Either way rows past
// the tensor repeat its last row: their scores are masked, so the finite
// values drop out.
template <int D, int NW>
struct Tile {
  using C = Cfg<D, NW>;
  static constexpr bool kDirect = D == 256;
  f32x4 x[kDirect ? 1 : C::NL];
  float* dst = nullptr;
  __device__ __forceinline__ void fetch(float* lds, const float* xp, int64_t xs, int r0, int rows, int tid) {
    if constexpr (kDirect) {
      constexpr int RPW = kTile / NW;  // rows per wave
      const int w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63;
#pragma unroll
      for (int i = 0; i < RPW; ++i) {
        const int r = w * RPW + i;
        const int n = min(r0 + r, rows - 1);
        load_lds16(xp + (int64_t)n * xs + 4 * l, lds_addr_of(lds + r * C::P));
      }
    } else {
      dst = lds;
#pragma unroll
      for (int i = 0; i < C::NL; ++i) {
        const int idx = tid + i * C::NT;
        const int r = idx / (D / 4), c = 4 * (idx % (D / 4));
        const int n = r0 + r;
        const int nc = n < rows ? n : rows - 1;
        x[i] = *(const f32x4*)(xp + (int64_t)nc * xs + c);
      }
    }
  }
  __device__ __forceinline__ void commit(int tid) const {
    if constexpr (!kDirect) {
#pragma unroll
      for (int i = 0; i < C::NL; ++i) {
        const int idx = tid + i * C::NT;
        if (C::N4 % C::NT == 0 || idx < C::N4) {
          const int r = idx / (D / 4), c = 4 * (idx % (D / 4));
          *(f32x4*)(dst + r * C::P + c) = x[i];
        }
      }
    }
  }
  __device__ static __forceinline__ void settle() {
    if constexpr (kDirect) wait_vmcnt<0>();
  }
};

__device__ __forceinline__ f32x4 lds4(const float* p) { return *(const f32x4*)p; }

// acc += A B^T over the head dim: A rows from LDS (row l32 of `t`, 16-byte
// reads one group of four MFMAs ahead), B from the lane's registers.
template <int HD, int P>
__device__ __forceinline__ void dsum(const float* t, const float (&b)[HD], f32x16& acc) {
  f32x4 cur = lds4(t);
#pragma unroll
  for (int k4 = 0; k4 < HD; k4 += 4) {
    f32x4 nxt = cur;
    if (k4 + 4 < HD) nxt = lds4(t + k4 + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = mma(cur[e], b[k4 + e], acc);
    cur = nxt;
    __builtin_amdgcn_sched_barrier(0);
  }
}
// acc[db] += A^T x over 32 rows: A column 32 db + l32 of `t` read at the rows
// of step r (one group of four steps ahead), x = the lane's element r.
template <int DB, int P>
__device__ __forceinline__ void rsum(const float* t, int l32, int h, const f32x16& x, f32x16 (&acc)[DB]) {
  float cur[4], nxt[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) cur[i] = t[blk_row(i, h) * P + l32];
#pragma unroll
  for (int g = 0; g < 4 * DB; ++g) {
    const int db = g >> 2, r0 = 4 * (g & 3);
#pragma unroll
    for (int i = 0; i < 4; ++i) nxt[i] = cur[i];
    if (g + 1 < 4 * DB) {
      const int db1 = (g + 1) >> 2, r1 = 4 * ((g + 1) & 3);
#pragma unroll
      for (int i = 0; i < 4; ++i) nxt[i] = t[blk_row(r1 + i, h) * P + 32 * db1 + l32];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[db] = mma(cur[i], x[r0 + i], acc[db]);
#pragma unroll
    for (int i = 0; i < 4; ++i) cur[i] = nxt[i];
    __builtin_amdgcn_sched_barrier(0);
  }
}
// --- 16 x 16 x 4 fp32 MFMA (16 accumulator columns per wave) -----------------
//   A operand  lane l holds A[row = l%16][k = l/16]
//   B operand  lane l holds B[k = l/16][col = l%16]
//   C/D        acc[r] = C[row = 4*(l/16) + r][col = l%16]
// Head-dim sums: lane group g = l/16 takes d = g*D/4 + s at step s.  16-row
// sums: at step s group g takes row 4g + s, the row of its accumulator
// element s.
__device__ __forceinline__ f32x4 mma16(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
// acc1 += A1 B1^T and acc2 += A2 B2^T over the head dim (A rows from LDS,
// 16-byte reads one group of four MFMAs ahead; B from registers).
template <int HD4>
__device__ __forceinline__ void dsum16x2(const float* t1, const float (&b1)[HD4], f32x4& acc1, const float* t2,
                                         const float (&b2)[HD4], f32x4& acc2) {
  f32x4 c1 = lds4(t1), c2 = lds4(t2);
#pragma unroll
  for (int k4 = 0; k4 < HD4; k4 += 4) {
    f32x4 n1 = c1, n2 = c2;
    if (k4 + 4 < HD4) {
      n1 = lds4(t1 + k4 + 4);
      n2 = lds4(t2 + k4 + 4);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc1 = mma16(c1[e], b1[k4 + e], acc1);
      acc2 = mma16(c2[e], b2[k4 + e], acc2);
    }
    c1 = n1;
    c2 = n2;
    __builtin_amdgcn_sched_barrier(0);
  }
}
// acc1[db] += A1^T x1 and acc2[db] += A2^T x2 over the 32 rows of a tile
// (two 16-row blocks qb): A column 16 db + l16 of t1 / t2 at row
// 16 qb + 4 g + s, x = the lane's element s of block qb.
template <int DB16, int P>
__device__ __forceinline__ void rsum16x2(const float* t1, const f32x4 (&x1)[2], f32x4 (&acc1)[DB16],
                                         const float* t2, const f32x4 (&x2)[2], f32x4 (&acc2)[DB16], int l16,
                                         int g) {
  constexpr int NG = 2 * DB16;  // groups of four MFMA steps: (db, qb)
  float c1[4], c2[4], n1[4], n2[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    c1[i] = t1[(4 * g + i) * P + l16];
    c2[i] = t2[(4 * g + i) * P + l16];
  }
#pragma unroll
  for (int q = 0; q < NG; ++q) {
    const int db = q >> 1, qb = q & 1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      n1[i] = c1[i];
      n2[i] = c2[i];
    }
    if (q + 1 < NG) {
      const int db1 = (q + 1) >> 1, qb1 = (q + 1) & 1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int off = (16 * qb1 + 4 * g + i) * P + 16 * db1 + l16;
        n1[i] = t1[off];
        n2[i] = t2[off];
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc1[db] = mma16(c1[i], x1[qb][i], acc1[db]);
      acc2[db] = mma16(c2[i], x2[qb][i], acc2[db]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      c1[i] = n1[i];
      c2[i] = n2[i];
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// acc[db] += A^T x over the 32 rows of a tile (two 16-row blocks qb): A
// column 16 db + l16 of t at row 16 qb + 4 g + s, x = the lane's element s
// of block qb.
template <int DB16, int P>
__device__ __forceinline__ void rsum16(const float* t, const f32x4 (&x)[2], f32x4 (&acc)[DB16], int l16, int g) {
  constexpr int NG = 2 * DB16;
  float c[4], n[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = t[(4 * g + i) * P + l16];
#pragma unroll
  for (int q = 0; q < NG; ++q) {
    const int db = q >> 1, qb = q & 1;
#pragma unroll
    for (int i = 0; i < 4; ++i) n[i] = c[i];
    if (q + 1 < NG) {
      const int db1 = (q + 1) >> 1, qb1 = (q + 1) & 1;
#pragma unroll
      for (int i = 0; i < 4; ++i) n[i] = t[(16 * qb1 + 4 * g + i) * P + 16 * db1 + l16];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[db] = mma16(c[i], x[qb][i], acc[db]);
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = n[i];
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Natural-domain transformed score (scale, soft-cap, ALiBi); t receives
// tanh(scale s / cap) for the soft-cap derivative.
template <bool SOFTCAP, bool ALIBI>
__device__ __forceinline__ float score(float s, const Shape& p, float slope, int i, int j, float& t) {
  float x = s * p.scale;
  if constexpr (SOFTCAP) {
    t = tanhf(x * p.inv_cap);
    x = p.cap * t;
  }
  if constexpr (ALIBI) x += slope * (float)(i - j);
  return x;
}

}  // namespace f32m

// ---------------------------------------------------------------------------
// Forward: each wave owns 32 query rows (the accumulator columns); the
// workgroup streams 32-row K/V tiles.
template <int D>
struct F32Fwd {
  static constexpr int NW = D == 256 ? 4 : 8;
  static constexpr int WPE = D == 256 ? 1 : (D == 128 ? 2 : 4);
  static constexpr int BM = 32 * NW;  // query rows per workgroup
};

// BLK: with a block map, the workgroup walks only the 32-key tiles whose
// 128 x 128 block is computed for some of its rows (a list built in dynamic
// LDS at the start); a wave whose own block is removed skips the tile.
template <int D, bool SOFTCAP, bool ALIBI, bool BLK = false>
__global__ __launch_bounds__(F32Fwd<D>::NW * 64) __attribute__((amdgpu_waves_per_eu(F32Fwd<D>::WPE, F32Fwd<D>::WPE)))
void fwd_f32_kernel(FwdArgs a) {
  using namespace f32m;
  constexpr int NW = F32Fwd<D>::NW, BM = F32Fwd<D>::BM;
  using C = Cfg<D, NW>;
  __shared__ __attribute__((aligned(16))) float sK[2][C::TILE];
  __shared__ __attribute__((aligned(16))) float sV[2][C::TILE];
  const Shape& p = a.p;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, h = lane >> 5;
  const int nbh = p.B * p.Hq;
  int kq, bh;
  if (!xcd_lpt_item(blockIdx.x, a.nqt, nbh, kq, bh)) {
    kq = blockIdx.x / nbh;
    bh = blockIdx.x % nbh;
  }
  const int qt = a.nqt - 1 - kq;  // longest causal items first
  const int hq = bh % p.Hq, b = bh / p.Hq, hk = hq / p.G;
  const int m0 = qt * BM, mw = m0 + 32 * wave, my_m = mw + l32;
  const float* qp = (const float*)a.q.data + b * a.q.sb + hq * a.q.sh;
  const float* kp = (const float*)a.k.data + b * a.k.sb + hk * a.k.sh;
  const float* vp = (const float*)a.v.data + b * a.v.sb + hk * a.v.sh;

  // Q as the B operand of S^T = K Q^T: lane holds Q[my_m][h*D/2 + s].
  float q[C::HD];
  {
    const int rq = min(my_m, p.Sq - 1);
    const float* src = qp + (int64_t)rq * a.q.ss + h * C::HD;
#pragma unroll
    for (int s = 0; s < C::HD; s += 4) {
      const f32x4 x = *(const f32x4*)(src + s);
#pragma unroll
      for (int e = 0; e < 4; ++e) q[s + e] = my_m < p.Sq ? x[e] : 0.f;
    }
  }
  const float slope = ALIBI ? p.alibi[hq] : 0.f;

  // KV range of the workgroup, of this wave, and the key interval of this row.
  int kv_lo = 0, kv_hi = p.Skv;
  if (p.causal) kv_hi = min(kv_hi, m0 + BM);
  if (p.window > 0) kv_lo = max(0, m0 - p.window);
  const int mlast = min(mw + 31, p.Sq - 1);
  const bool wave_live = mw < p.Sq;
  int w_lo = kv_lo, w_hi = kv_hi;
  if (p.causal) w_hi = min(w_hi, mlast + 1);
  if (p.window > 0) w_lo = max(w_lo, mw - p.window);
  if (p.doc) {
    int l0, h0, l1, h1;
    doc_bounds(p, b, min(m0, p.Sq - 1), l0, h0);
    doc_bounds(p, b, min(m0 + BM, p.Sq) - 1, l1, h1);
    kv_lo = max(kv_lo, l0);
    kv_hi = min(kv_hi, h1);
    doc_bounds(p, b, min(mw, p.Sq - 1), l0, h0);
    doc_bounds(p, b, mlast, l1, h1);
    w_lo = max(w_lo, l0);
    w_hi = min(w_hi, h1);
  }
  int row_lo, row_hi;
  doc_bounds(p, b, min(my_m, p.Sq - 1), row_lo, row_hi);
  row_lo = max(row_lo, 0);
  row_hi = min(row_hi, p.Skv);
  if (p.causal) row_hi = min(row_hi, my_m + 1);
  if (p.window > 0) row_lo = max(row_lo, my_m - p.window);
  const unsigned row_w = (unsigned)max(row_hi - row_lo, 0);
  const unsigned char* brow = p.blk && wave_live ? block_row(p, b, hq, mw) : nullptr;

  f32x16 acc[C::DB];
#pragma unroll
  for (int db = 0; db < C::DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
  float m_run = kNegInf, l_run = 0.f;  // l_run: this lane's half of the row sum

  Tile<D, NW> st;
  const int n_first = (kv_lo / kTile) * kTile;
  int nv = max((kv_hi - n_first + kTile - 1) / kTile, 0);  // tiles walked
  extern __shared__ unsigned short tlist[];  // BLK: walk position -> tile offset from n_first
  __shared__ int s_nv;
  if (BLK && nv > 0) {
    if (wave == 0) {
      const int rb0 = m0 / kBlk, rb1 = (min(m0 + BM, p.Sq) - 1) / kBlk;  // the workgroup's block rows
      int base = 0;
      for (int i0 = 0; i0 < nv; i0 += 64) {
        const int i = i0 + lane;
        bool live = false;
        if (i < nv) {
          const int kb = (n_first + kTile * i) / kBlk;
          for (int rb = rb0; rb <= rb1 && !live; ++rb) live = block_row(p, b, hq, rb * kBlk)[kb] != 0;
        }
        const unsigned long long msk = __builtin_amdgcn_ballot_w64(live);
        if (live) tlist[base + __builtin_popcountll(msk & ((1ull << lane) - 1))] = (unsigned short)i;
        base += __builtin_popcountll(msk);
      }
      if (lane == 0) s_nv = base;
    }
    __syncthreads();
    nv = __builtin_amdgcn_readfirstlane(s_nv);
  }
  auto tile_n0 = [&](int v) -> int {
    if constexpr (BLK) return n_first + kTile * __builtin_amdgcn_readfirstlane((int)tlist[v]);
    else return n_first + kTile * v;
  };
  if (nv > 0) {
    st.fetch(sK[0], kp, a.k.ss, tile_n0(0), p.Skv, tid);
    st.commit(tid);
    st.fetch(sV[0], vp, a.v.ss, tile_n0(0), p.Skv, tid);
    st.commit(tid);
  }
  st.settle();
  __syncthreads();
  int buf = 0;
  for (int v = 0; v < nv; ++v, buf ^= 1) {
    const int n0 = tile_n0(v);
    const bool more = v + 1 < nv;
    const int n1 = more ? tile_n0(v + 1) : 0;
    const bool on = wave_live && n0 < w_hi && n0 + kTile > w_lo && (!brow || brow[n0 / kBlk] != 0);
    // next K tile in flight during this tile's S^T, next V tile during its P V
    if (more) st.fetch(sK[buf ^ 1], kp, a.k.ss, n1, p.Skv, tid);
    f32x16 s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
    if (on) dsum<C::HD, C::P>(sK[buf] + l32 * C::P + h * C::HD, q, s);
    if (more) {
      st.commit(tid);
      st.fetch(sV[buf ^ 1], vp, a.v.ss, n1, p.Skv, tid);
    }
    if (on) {
      // scores, mask, online softmax over this lane's 16 keys and the other half's
      const int a0 = row_lo - n0 - 4 * h;
      float mx = kNegInf;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int j = n0 + blk_row(r, h);
        float t;
        float x = score<SOFTCAP, ALIBI>(s[r], p, slope, my_m, j, t);
        if ((unsigned)(8 * (r >> 2) + (r & 3) - a0) >= row_w) x = kNegInf;
        s[r] = x;
        mx = fmaxf(mx, x);
      }
      mx = fmaxf(mx, swap_halves(mx));
      const float m_new = fmaxf(m_run, mx);
      const float m_use = m_new == kNegInf ? 0.f : m_new;
      const float alpha = expf(m_run - m_use);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < C::DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] = expf(s[r] - m_use);
        l_run += s[r];
      }
      m_run = m_new;
      // O^T += V^T P^T: A = V[row of step r][32 db + l32], B = P^T (element r)
      rsum<C::DB, C::P>(sV[buf], l32, h, s, acc);
    }
    if (more) st.commit(tid);
    st.settle();
    __syncthreads();
  }

  const float l_tot = l_run + swap_halves(l_run);
  if (my_m < p.Sq) {
    const bool empty = !(l_tot > 0.f);
    float* op = (float*)a.o.data + b * a.o.sb + hq * a.o.sh + (int64_t)my_m * a.o.ss;
#pragma unroll
    for (int db = 0; db < C::DB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = empty ? 0.f : acc[db][4 * i + e] / l_tot;
        *(f32x4*)(op + 32 * db + 8 * i + 4 * h) = v;
      }
    if (h == 0) a.lse[(int64_t)(b * p.Hq + hq) * p.Sq + my_m] = empty ? kNegInf : m_run + logf(l_tot);
  }
}

// ---------------------------------------------------------------------------
// dQ recomputing S and dP (the backward without a dS workspace): each wave
// owns 16 query rows (the accumulator columns of the 16 x 16 x 4 MFMA) and
// streams 32-row K/V tiles: S^T = K Q^T, dP^T = V dO^T, dQ^T += K^T dS^T.  Q,
// dO and dQ take D/4 values per lane: two waves per SIMD at D <= 128, one
// at D = 256.
template <int D>
struct F32Dq16 {
  static constexpr int NW = D == 256 ? 4 : 8;
  static constexpr int WPE = D == 256 ? 1 : 2;
  static constexpr int BM = 16 * NW;  // query rows per workgroup
};

template <int D, bool SOFTCAP, bool ALIBI>
__global__ __launch_bounds__(F32Dq16<D>::NW * 64)
__attribute__((amdgpu_waves_per_eu(F32Dq16<D>::WPE, F32Dq16<D>::WPE)))
void bwd_dq16_f32_kernel(BwdArgs a) {
  using namespace f32m;
  constexpr int NW = F32Dq16<D>::NW, BM = F32Dq16<D>::BM;
  constexpr int HD4 = D / 4, DB16 = D / 16;
  using C = Cfg<D, NW>;
  __shared__ __attribute__((aligned(16))) float sK[2][C::TILE];
  __shared__ __attribute__((aligned(16))) float sV[2][C::TILE];
  const Shape& p = a.p;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l16 = lane & 15, g = lane >> 4;
  const int nbh = p.B * p.Hq;
  int kq, bh;
  if (!xcd_lpt_item(blockIdx.x, a.ntiles, nbh, kq, bh)) {
    kq = blockIdx.x / nbh;
    bh = blockIdx.x % nbh;
  }
  const int qt = a.ntiles - 1 - kq;
  const int hq = bh % p.Hq, b = bh / p.Hq, hk = hq / p.G;
  const int m0 = qt * BM, mw = m0 + 16 * wave, my_m = mw + l16;
  const float* qp = (const float*)a.q.data + b * a.q.sb + hq * a.q.sh;
  const float* dop = (const float*)a.dout.data + b * a.dout.sb + hq * a.dout.sh;
  const float* kp = (const float*)a.k.data + b * a.k.sb + hk * a.k.sh;
  const float* vp = (const float*)a.v.data + b * a.v.sb + hk * a.v.sh;

  // Q and dO as the B operands of S^T = K Q^T and dP^T = V dO^T: Q[my_m][g*D/4 + s].
  float q[HD4], dO[HD4];
  {
    const int rq = min(my_m, p.Sq - 1);
    const float* s1 = qp + (int64_t)rq * a.q.ss + g * HD4;
    const float* s2 = dop + (int64_t)rq * a.dout.ss + g * HD4;
#pragma unroll
    for (int s = 0; s < HD4; s += 4) {
      const f32x4 x = *(const f32x4*)(s1 + s);
      const f32x4 y = *(const f32x4*)(s2 + s);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        q[s + e] = my_m < p.Sq ? x[e] : 0.f;
        dO[s + e] = my_m < p.Sq ? y[e] : 0.f;
      }
    }
  }
  float lse = kPosInf, dl = 0.f;
  if (my_m < p.Sq) {
    const int64_t ri = (int64_t)(b * p.Hq + hq) * p.Sq + my_m;
    lse = a.lse[ri] == kNegInf ? kPosInf : a.lse[ri];
    dl = a.delta[ri];
  }
  const float slope = ALIBI ? p.alibi[hq] : 0.f;

  int kv_lo = 0, kv_hi = p.Skv;
  if (p.causal) kv_hi = min(kv_hi, m0 + BM);
  if (p.window > 0) kv_lo = max(0, m0 - p.window);
  const int mlast = min(mw + 15, p.Sq - 1);
  const bool wave_live = mw < p.Sq;
  int w_lo = kv_lo, w_hi = kv_hi;
  if (p.causal) w_hi = min(w_hi, mlast + 1);
  if (p.window > 0) w_lo = max(w_lo, mw - p.window);
  if (p.doc) {
    int l0, h0, l1, h1;
    doc_bounds(p, b, min(m0, p.Sq - 1), l0, h0);
    doc_bounds(p, b, min(m0 + BM, p.Sq) - 1, l1, h1);
    kv_lo = max(kv_lo, l0);
    kv_hi = min(kv_hi, h1);
    doc_bounds(p, b, min(mw, p.Sq - 1), l0, h0);
    doc_bounds(p, b, mlast, l1, h1);
    w_lo = max(w_lo, l0);
    w_hi = min(w_hi, h1);
  }
  int row_lo, row_hi;
  doc_bounds(p, b, min(my_m, p.Sq - 1), row_lo, row_hi);
  row_lo = max(row_lo, 0);
  row_hi = min(row_hi, p.Skv);
  if (p.causal) row_hi = min(row_hi, my_m + 1);
  if (p.window > 0) row_lo = max(row_lo, my_m - p.window);
  const unsigned row_w = (unsigned)max(row_hi - row_lo, 0);
  const unsigned char* brow = p.blk && wave_live ? block_row(p, b, hq, mw) : nullptr;

  f32x4 acc[DB16];
#pragma unroll
  for (int db = 0; db < DB16; ++db)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[db][r] = 0.f;

  Tile<D, NW> sk, sv;
  const int n_first = (kv_lo / kTile) * kTile;
  if (n_first < kv_hi) {
    sk.fetch(sK[0], kp, a.k.ss, n_first, p.Skv, tid);
    sv.fetch(sV[0], vp, a.v.ss, n_first, p.Skv, tid);
    sk.commit(tid);
    sv.commit(tid);
  }
  sk.settle();
  __syncthreads();
  int buf = 0;
  for (int n0 = n_first; n0 < kv_hi; n0 += kTile, buf ^= 1) {
    const bool more = n0 + kTile < kv_hi;
    if (more) {
      sk.fetch(sK[buf ^ 1], kp, a.k.ss, n0 + kTile, p.Skv, tid);
      sv.fetch(sV[buf ^ 1], vp, a.v.ss, n0 + kTile, p.Skv, tid);
    }
    const bool on = wave_live && n0 < w_hi && n0 + kTile > w_lo && (!brow || brow[n0 / kBlk] != 0);
    if (on) {
      f32x4 s[2], dp[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) s[kb][r] = dp[kb][r] = 0.f;
        const int ro = (16 * kb + l16) * C::P + g * HD4;
        dsum16x2<HD4>(sK[buf] + ro, q, s[kb], sV[buf] + ro, dO, dp[kb]);
      }
      // element (kb, r): key n0 + 16 kb + 4 g + r of query row my_m
      const int a0 = row_lo - n0 - 4 * g;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = n0 + 16 * kb + 4 * g + r;
          float t = 0.f;
          const float x = score<SOFTCAP, ALIBI>(s[kb][r], p, slope, my_m, j, t);
          const float pj = (unsigned)(16 * kb + r - a0) < row_w ? expf(x - lse) : 0.f;
          float ds = pj * (dp[kb][r] - dl) * p.scale;
          if constexpr (SOFTCAP) ds *= (1.0f - t * t);
          s[kb][r] = ds;
        }
      // dQ^T += K^T dS^T over the tile's 32 keys
      rsum16<DB16, C::P>(sK[buf], s, acc, l16, g);
    }
    if (more) {
      sk.commit(tid);
      sv.commit(tid);
    }
    sk.settle();
    __syncthreads();
  }
  if (my_m < p.Sq) {
    float* op = (float*)a.dq.data + b * a.dq.sb + hq * a.dq.sh + (int64_t)my_m * a.dq.ss;
#pragma unroll
    for (int db = 0; db < DB16; ++db) *(f32x4*)(op + 16 * db + 4 * g) = acc[db];
  }
}

// ---------------------------------------------------------------------------
// dK/dV: each wave owns 16 KV rows (the accumulator columns of the
// 16 x 16 x 4 MFMA) and streams 32-row Q/dO tiles of every query head of
// its group: S = Q K^T, dP = dO V^T, dV^T += dO^T P, dK^T += Q^T dS.  K, V,
// dK and dV take D/4 values per lane, so two waves share a SIMD at
// D <= 128 and D = 256 fits one wave's registers (32 KV rows per wave on the
// 32 x 32 x 2 MFMA need D/2 each: one wave per SIMD at D = 128, 1.3x
// slower).  With DS the kernel also stores the dS it feeds dK into the
// staged-dS units: every (query tile, 128-row block) unit of the causal /
// window band that its rows fall in, zeros where a wave skips or masks.
template <int D>
struct F32Kv16 {
  static constexpr int NW = D == 256 ? 4 : 8;
  static constexpr int WPE = D == 256 ? 1 : 2;
  static constexpr int BN = 16 * NW;  // KV rows per workgroup
};

template <int D, bool SOFTCAP, bool ALIBI, bool DS>
__global__ __launch_bounds__(F32Kv16<D>::NW * 64)
__attribute__((amdgpu_waves_per_eu(F32Kv16<D>::WPE, F32Kv16<D>::WPE)))
void bwd_dkdv16_f32_kernel(BwdArgs a) {
  using namespace f32m;
  constexpr int NW = F32Kv16<D>::NW, BN = F32Kv16<D>::BN;
  constexpr int HD4 = D / 4, DB16 = D / 16;
  using C = Cfg<D, NW>;
  __shared__ __attribute__((aligned(16))) float sQ[2][C::TILE];
  __shared__ __attribute__((aligned(16))) float sO[2][C::TILE];
  __shared__ __attribute__((aligned(16))) float sL[2][kTile];
  __shared__ __attribute__((aligned(16))) float sDl[2][kTile];
  const Shape& p = a.p;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l16 = lane & 15, g = lane >> 4;
  const int nbh = p.B * p.Hkv;
  int kt, bh;
  if (!xcd_lpt_item(blockIdx.x, a.ntiles, nbh, kt, bh)) {  // causal: low KV tiles are the longest
    kt = blockIdx.x / nbh;
    bh = blockIdx.x % nbh;
  }
  const int hk = bh % p.Hkv, b = bh / p.Hkv;
  const int n0 = kt * BN, nw = n0 + 16 * wave, my_n = nw + l16;
  const float* kp = (const float*)a.k.data + b * a.k.sb + hk * a.k.sh;
  const float* vp = (const float*)a.v.data + b * a.v.sb + hk * a.v.sh;

  // K and V as the B operands of S = Q K^T and dP = dO V^T: K[my_n][g*D/4 + s].
  float kr[HD4], vr[HD4];
  {
    const int rn = min(my_n, p.Skv - 1);
    const float* s1 = kp + (int64_t)rn * a.k.ss + g * HD4;
    const float* s2 = vp + (int64_t)rn * a.v.ss + g * HD4;
#pragma unroll
    for (int s = 0; s < HD4; s += 4) {
      const f32x4 x = *(const f32x4*)(s1 + s);
      const f32x4 y = *(const f32x4*)(s2 + s);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kr[s + e] = my_n < p.Skv ? x[e] : 0.f;
        vr[s + e] = my_n < p.Skv ? y[e] : 0.f;
      }
    }
  }

  // Query range of the workgroup, of this wave, and the query interval of this KV row.
  int q_lo = p.causal ? n0 : 0, q_hi = p.Sq;
  if (p.window > 0) q_hi = min(q_hi, n0 + BN + p.window);
  if constexpr (DS) {  // the whole band of the 128-row dS blocks the workgroup's rows fall in
    if (p.causal) q_lo = kDsKB * (n0 / kDsKB);
    if (p.window > 0) q_hi = min(p.Sq, kDsKB * ((n0 + BN - 1) / kDsKB + 1) + p.window);
  }
  const int nlast = min(nw + 15, p.Skv - 1);
  const bool wave_live = nw < p.Skv;
  int w_lo = q_lo, w_hi = q_hi;
  if (p.causal) w_lo = max(w_lo, nw);
  if (p.window > 0) w_hi = min(w_hi, nlast + p.window + 1);
  if (p.docc) {
    int l0, h0, l1, h1;
    if constexpr (!DS) {  // DS: every query tile of the causal / window band is visited (and its dS stored)
      col_bounds(p, b, min(n0, p.Skv - 1), l0, h0);
      col_bounds(p, b, min(n0 + BN, p.Skv) - 1, l1, h1);
      q_lo = max(q_lo, l0);
      q_hi = min(q_hi, h1);
    }
    col_bounds(p, b, min(nw, p.Skv - 1), l0, h0);
    col_bounds(p, b, nlast, l1, h1);
    w_lo = max(w_lo, l0);
    w_hi = min(w_hi, h1);
  }
  int col_lo, col_hi;
  col_bounds(p, b, min(my_n, p.Skv - 1), col_lo, col_hi);
  col_lo = max(col_lo, 0);
  col_hi = min(col_hi, p.Sq);
  if (p.causal) col_lo = max(col_lo, my_n);
  if (p.window > 0) col_hi = min(col_hi, my_n + p.window + 1);
  if (my_n >= p.Skv) col_hi = col_lo;
  const unsigned col_w = (unsigned)max(col_hi - col_lo, 0);

  f32x4 dk[DB16], dv[DB16];
#pragma unroll
  for (int db = 0; db < DB16; ++db)
#pragma unroll
    for (int r = 0; r < 4; ++r) dk[db][r] = dv[db][r] = 0.f;

  // Staged dS: this wave's 128-row KV block and its column offset in the block.
  const int nkb = (p.Skv + kDsKB - 1) / kDsKB;
  const int kb_w = nw / kDsKB, j_w = nw % kDsKB + l16;

  const int m_first = (q_lo / kTile) * kTile;
  const int nq = q_hi > m_first ? (q_hi - m_first + kTile - 1) / kTile : 0;  // query tiles per head
  const int total = nq * p.G;
  Tile<D, NW> st;
  float lv = 0.f, dv0 = 0.f;  // LSE and Delta of one query row (threads < 32)
  auto step_ptrs = [&](int u, const float*& qp, const float*& dop, int& m, int& hq) {
    const int gg = u / nq;
    m = m_first + kTile * (u % nq);
    hq = hk * p.G + gg;
    qp = (const float*)a.q.data + b * a.q.sb + hq * a.q.sh;
    dop = (const float*)a.dout.data + b * a.dout.sb + hq * a.dout.sh;
  };
  auto load_rows = [&](int m, int hq) {
    if (tid < kTile) {
      const int mi = m + tid;
      lv = kPosInf;
      dv0 = 0.f;
      if (mi < p.Sq) {
        const int64_t ri = (int64_t)(b * p.Hq + hq) * p.Sq + mi;
        lv = a.lse[ri] == kNegInf ? kPosInf : a.lse[ri];
        dv0 = a.delta[ri];
      }
    }
  };
  auto store_rows = [&](int bf) {
    if (tid < kTile) {
      sL[bf][tid] = lv;
      sDl[bf][tid] = dv0;
    }
  };
  if (total > 0) {
    const float *qp, *dop;
    int m, hq;
    step_ptrs(0, qp, dop, m, hq);
    st.fetch(sQ[0], qp, a.q.ss, m, p.Sq, tid);
    st.commit(tid);
    st.fetch(sO[0], dop, a.dout.ss, m, p.Sq, tid);
    st.commit(tid);
    load_rows(m, hq);
    store_rows(0);
  }
  st.settle();
  __syncthreads();
  int buf = 0;
  for (int u = 0; u < total; ++u, buf ^= 1) {
    const bool more = u + 1 < total;
    const float *nqp = nullptr, *ndop = nullptr;
    int nm = 0, nhq = 0;
    if (more) {
      step_ptrs(u + 1, nqp, ndop, nm, nhq);
      st.fetch(sQ[buf ^ 1], nqp, a.q.ss, nm, p.Sq, tid);
      load_rows(nm, nhq);
    }
    const int m0 = m_first + kTile * (u % nq);
    const int hq = hk * p.G + u / nq;
    const bool on = wave_live && m0 < w_hi && m0 + kTile > w_lo &&
                    (!p.blk || block_row(p, b, hq, m0)[nw / kBlk] != 0);
    f32x4 s[2], dp[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int r = 0; r < 4; ++r) s[qb][r] = dp[qb][r] = 0.f;
    if (on) {
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const int ro = (16 * qb + l16) * C::P + g * HD4;
        dsum16x2<HD4>(sQ[buf] + ro, kr, s[qb], sO[buf] + ro, vr, dp[qb]);
      }
    }
    if (more) {
      st.commit(tid);
      st.fetch(sO[buf ^ 1], ndop, a.dout.ss, nm, p.Sq, tid);
    }
    if (on) {
      const float slope = ALIBI ? p.alibi[hq] : 0.f;
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const f32x4 l4 = lds4(&sL[buf][16 * qb + 4 * g]);
        const f32x4 d4 = lds4(&sDl[buf][16 * qb + 4 * g]);
        const int a0 = col_lo - m0 - 16 * qb - 4 * g;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int mi = m0 + 16 * qb + 4 * g + r;
          float t = 0.f;
          const float x = score<SOFTCAP, ALIBI>(s[qb][r], p, slope, mi, my_n, t);
          const float pj = (unsigned)(r - a0) < col_w ? expf(x - l4[r]) : 0.f;
          float d = pj * (dp[qb][r] - d4[r]) * p.scale;
          if constexpr (SOFTCAP) d *= (1.0f - t * t);
          s[qb][r] = pj;
          dp[qb][r] = d;
        }
      }
      // dV^T += dO^T P and dK^T += Q^T dS over the tile's 32 query rows
      rsum16x2<DB16, C::P>(sO[buf], s, dv, sQ[buf], dp, dk, l16, g);
    }
    if constexpr (DS) {
      // units of removed blocks are neither written nor read (their dS is zero)
      const int t = m0 / kDsQT;
      const int kb_lo = ds_kb_lo(t, p.window, nkb);
      if (kb_w < nkb && kb_w >= kb_lo && kb_w < ds_kb_hi(t, p.causal, nkb) &&
          (!p.blk || block_row(p, b, hq, min(m0, p.Sq - 1))[kb_w] != 0)) {
        const int64_t unit = (int64_t)(b * p.Hq + hq) * a.ds_head + ds_tile_offset(t, p.causal, p.window, nkb) +
                             (kb_w - kb_lo);
        // element (query row i, KV column j) of the unit at ((j / 32) * 32 + i) * 32 + j % 32
        float* dst = (float*)(a.ds + unit * kDsUnitB32) + (j_w / kTile) * (kTile * kTile) + j_w % kTile;
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int r = 0; r < 4; ++r) __builtin_nontemporal_store(dp[qb][r], dst + (16 * qb + 4 * g + r) * kTile);
      }
    }
    if (more) {
      st.commit(tid);
      store_rows(buf ^ 1);
    }
    st.settle();
    __syncthreads();
  }
  if (my_n < p.Skv) {
    float* kd = (float*)a.dk.data + b * a.dk.sb + hk * a.dk.sh + (int64_t)my_n * a.dk.ss;
    float* vd = (float*)a.dv.data + b * a.dv.sb + hk * a.dv.sh + (int64_t)my_n * a.dv.ss;
#pragma unroll
    for (int db = 0; db < DB16; ++db) {
      *(f32x4*)(kd + 16 * db + 4 * g) = dk[db];
      *(f32x4*)(vd + 16 * db + 4 * g) = dv[db];
    }
  }
}

// ---------------------------------------------------------------------------
// dQ = dS K from the fp32 dS the dK/dV kernel staged (no S or dP recompute):
// each wave owns 32 query rows (one dS unit row band) and streams 32-row K
// tiles over the band of KV blocks of its query tile.
template <int D>
struct F32DqDs {
  static constexpr int NW = 8;
  static constexpr int WPE = 2;
  static constexpr int BM = 32 * NW;
};

template <int D>
__global__ __launch_bounds__(F32DqDs<D>::NW * 64) __attribute__((amdgpu_waves_per_eu(F32DqDs<D>::WPE, F32DqDs<D>::WPE)))
void bwd_dq_ds_f32_kernel(BwdArgs a) {
  using namespace f32m;
  constexpr int NW = F32DqDs<D>::NW, BM = F32DqDs<D>::BM;
  using C = Cfg<D, NW>;
  __shared__ __attribute__((aligned(16))) float sK[2][C::TILE];
  const Shape& p = a.p;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, h = lane >> 5;
  const int nbh = p.B * p.Hq;
  int kq, bh;
  if (!xcd_lpt_item(blockIdx.x, a.ntiles, nbh, kq, bh)) {
    kq = blockIdx.x / nbh;
    bh = blockIdx.x % nbh;
  }
  const int qt = a.ntiles - 1 - kq;
  const int hq = bh % p.Hq, b = bh / p.Hq, hk = hq / p.G;
  const int m0 = qt * BM, mw = m0 + 32 * wave, my_m = mw + l32;
  const float* kp = (const float*)a.k.data + b * a.k.sb + hk * a.k.sh;
  const int nkb = (p.Skv + kDsKB - 1) / kDsKB;

  // KV blocks of this wave's query tile, and of the workgroup's tiles
  const bool wave_live = mw < p.Sq;
  const int t = mw / kDsQT;
  const int w_kb_lo = ds_kb_lo(t, p.window, nkb), w_kb_hi = wave_live ? ds_kb_hi(t, p.causal, nkb) : 0;
  const int t_first = m0 / kDsQT, t_last = (min(m0 + BM, p.Sq) - 1) / kDsQT;
  const int kv_lo = kDsKB * ds_kb_lo(t_first, p.window, nkb);
  const int kv_hi = min(p.Skv, kDsKB * ds_kb_hi(t_last, p.causal, nkb));
  // unit of block kb for this wave: ubase + kb
  const int64_t ubase = (int64_t)(b * p.Hq + hq) * a.ds_head + ds_tile_offset(t, p.causal, p.window, nkb) - w_kb_lo;
  const float* dsb = (const float*)a.ds + l32 * kTile + 4 * h;
  // block maps: the units of this wave's removed blocks are not read (never written, their dS is zero)
  const unsigned char* brow = p.blk && wave_live ? block_row(p, b, hq, mw) : nullptr;
  auto unit_live = [&](int kb) { return kb >= w_kb_lo && kb < w_kb_hi && (!brow || brow[kb] != 0); };

  f32x16 acc[C::DB];
#pragma unroll
  for (int db = 0; db < C::DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;

  // dS^T operand of one 32-row K tile: element r = dS[my_m][n0 + row of step r]
  auto load_ds = [&](int n0, f32x16& x) {
    const int kb = n0 / kDsKB;
    if (unit_live(kb)) {
      const float* src = dsb + (ubase + kb) * (kDsUnitB32 / 4) + ((n0 % kDsKB) / kTile) * (kTile * kTile);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 v = *(const f32x4*)(src + 8 * j);
#pragma unroll
        for (int e = 0; e < 4; ++e) x[4 * j + e] = v[e];
      }
    }
  };

  Tile<D, NW> st;
  f32x16 cur, nxt;
#pragma unroll
  for (int r = 0; r < 16; ++r) cur[r] = nxt[r] = 0.f;
  if (kv_lo < kv_hi) {
    st.fetch(sK[0], kp, a.k.ss, kv_lo, p.Skv, tid);
    load_ds(kv_lo, cur);
    st.commit(tid);
  }
  st.settle();
  __syncthreads();
  int buf = 0;
  for (int n0 = kv_lo; n0 < kv_hi; n0 += kTile, buf ^= 1) {
    const bool more = n0 + kTile < kv_hi;
    if (more) {
      st.fetch(sK[buf ^ 1], kp, a.k.ss, n0 + kTile, p.Skv, tid);
      load_ds(n0 + kTile, nxt);
    }
    if (unit_live(n0 / kDsKB)) rsum<C::DB, C::P>(sK[buf], l32, h, cur, acc);
    if (more) st.commit(tid);
    st.settle();
    __syncthreads();
    cur = nxt;
  }
  if (my_m < p.Sq) {
    float* op = (float*)a.dq.data + b * a.dq.sb + hq * a.dq.sh + (int64_t)my_m * a.dq.ss;
#pragma unroll
    for (int db = 0; db < C::DB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[db][4 * i + e];
        *(f32x4*)(op + 32 * db + 8 * i + 4 * h) = v;
      }
  }
}

// The four (soft-cap, ALiBi) instances of a kernel.
#define FLEXATT_F32_LAUNCH(kern, grid, block, st, x)                                           \
  do {                                                                                          \
    const bool sc_ = (x).p.cap > 0.f, al_ = (x).p.alibi != nullptr;                             \
    if (sc_ && al_) hipLaunchKernelGGL((kern<FLEXATT_D, true, true>), grid, block, 0, st, x);   \
    else if (sc_) hipLaunchKernelGGL((kern<FLEXATT_D, true, false>), grid, block, 0, st, x);    \
    else if (al_) hipLaunchKernelGGL((kern<FLEXATT_D, false, true>), grid, block, 0, st, x);    \
    else hipLaunchKernelGGL((kern<FLEXATT_D, false, false>), grid, block, 0, st, x);            \
  } while (0)

// The same with a fourth template argument.
#define FLEXATT_F32_LAUNCH4(kern, X, grid, block, st, x)                                            \
  do {                                                                                              \
    const bool sc_ = (x).p.cap > 0.f, al_ = (x).p.alibi != nullptr;                                 \
    if (sc_ && al_) hipLaunchKernelGGL((kern<FLEXATT_D, true, true, X>), grid, block, 0, st, x);    \
    else if (sc_) hipLaunchKernelGGL((kern<FLEXATT_D, true, false, X>), grid, block, 0, st, x);     \
    else if (al_) hipLaunchKernelGGL((kern<FLEXATT_D, false, true, X>), grid, block, 0, st, x);     \
    else hipLaunchKernelGGL((kern<FLEXATT_D, false, false, X>), grid, block, 0, st, x);             \
  } while (0)

#define FLEXATT_CAT2(a, b) a##b
#define FLEXATT_CAT(a, b) FLEXATT_CAT2(a, b)

hipError_t FLEXATT_CAT(fwd_f32_d, FLEXATT_D)(const FwdArgs& a, hipStream_t st) {
  using F = F32Fwd<FLEXATT_D>;
  FwdArgs x = a;
  x.nqt = (a.p.Sq + F::BM - 1) / F::BM;
  const dim3 grid(x.nqt * a.p.B * a.p.Hq), block(F::NW * 64);
  // block maps: the walk list of live 32-key tiles in dynamic LDS (up to
  // 16 KB beside the tiles; longer key ranges walk every tile)
  const size_t dyn = 2 * (size_t)((a.p.Skv + f32m::kTile - 1) / f32m::kTile + 2);
  if (a.p.blk && dyn <= 16384) {
    const bool sc = a.p.cap > 0.f, al = a.p.alibi != nullptr;
    if (sc && al) hipLaunchKernelGGL((fwd_f32_kernel<FLEXATT_D, true, true, true>), grid, block, dyn, st, x);
    else if (sc) hipLaunchKernelGGL((fwd_f32_kernel<FLEXATT_D, true, false, true>), grid, block, dyn, st, x);
    else if (al) hipLaunchKernelGGL((fwd_f32_kernel<FLEXATT_D, false, true, true>), grid, block, dyn, st, x);
    else hipLaunchKernelGGL((fwd_f32_kernel<FLEXATT_D, false, false, true>), grid, block, dyn, st, x);
    return hipGetLastError();
  }
  FLEXATT_F32_LAUNCH(fwd_f32_kernel, grid, block, st, x);
  return hipGetLastError();
}

hipError_t FLEXATT_CAT(bwd_dq_f32_d, FLEXATT_D)(const BwdArgs& a, hipStream_t st) {
  using F = F32Dq16<FLEXATT_D>;
  BwdArgs x = a;
  x.ntiles = (a.p.Sq + F::BM - 1) / F::BM;
  FLEXATT_F32_LAUNCH(bwd_dq16_f32_kernel, dim3(x.ntiles * a.p.B * a.p.Hq), dim3(F::NW * 64), st, x);
  return hipGetLastError();
}
hipError_t FLEXATT_CAT(bwd_dkdv_f32_d, FLEXATT_D)(const BwdArgs& a, hipStream_t st) {
  using F = F32Kv16<FLEXATT_D>;
  BwdArgs x = a;
  x.ntiles = (a.p.Skv + F::BN - 1) / F::BN;
  FLEXATT_F32_LAUNCH4(bwd_dkdv16_f32_kernel, false, dim3(x.ntiles * a.p.B * a.p.Hkv), dim3(F::NW * 64), st, x);
  return hipGetLastError();
}
hipError_t FLEXATT_CAT(bwd_kv_ds_f32_d, FLEXATT_D)(const BwdArgs& a, hipStream_t st) {
  using F = F32Kv16<FLEXATT_D>;
  BwdArgs x = a;
  x.ntiles = (a.p.Skv + F::BN - 1) / F::BN;
  FLEXATT_F32_LAUNCH4(bwd_dkdv16_f32_kernel, true, dim3(x.ntiles * a.p.B * a.p.Hkv), dim3(F::NW * 64), st, x);
  return hipGetLastError();
}
hipError_t FLEXATT_CAT(bwd_dq_ds_f32_d, FLEXATT_D)(const BwdArgs& a, hipStream_t st) {
  using F = F32DqDs<FLEXATT_D>;
  BwdArgs x = a;
  x.ntiles = (a.p.Sq + F::BM - 1) / F::BM;
  hipLaunchKernelGGL((bwd_dq_ds_f32_kernel<FLEXATT_D>), dim3(x.ntiles * a.p.B * a.p.Hq), dim3(F::NW * 64), 0, st, x);
  return hipGetLastError();
}

}  // namespace flexatt
