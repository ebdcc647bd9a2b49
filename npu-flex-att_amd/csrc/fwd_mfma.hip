// Flash-attention forward for fp16/bf16 on gfx950 MFMA.
//
// Semantics: npu_flash_attention.py:17-166 (flash_attn_fwd_kernel) — online
// softmax over KV tiles, O in the input dtype, LSE in fp32 natural log, the
// score order scale -> soft-cap -> ALiBi -> mask, GQA head h -> h / G.
//
// Decomposition
//  * One workgroup = NW waves = one (batch, KV head) pair, a group of gp query
//    heads that share that KV head (gp = the largest power of two dividing G,
//    at most NW), and 32 * NW / gp query rows of each of them.  Every K/V tile
//    brought on chip therefore serves gp heads at once (GQA is indexed
//    directly: no K/V expansion, and gp times less L2->LDS traffic).
//  * Each wave owns 32 query rows of one head and computes S^T = K Q^T per
//    32x32 block (A = K rows from LDS, B = its Q rows held in registers), so
//    every lane holds one query row: the row max needs one exchange between
//    the two wave halves and the O rescale is a per-lane scalar.
//  * O^T = V^T P^T, with P^T taken straight from the S^T accumulators and V^T
//    read from the row-major V tile with the LDS transpose read.
//  * K/V tiles are copied global -> LDS with direct-to-LDS loads (no staging
//    registers): into four stages three tiles ahead with the 8-wave
//    ping-pong (one barrier per phase), into three stages two tiles ahead
//    with 4 waves (one barrier per tile).  Tiles are unpadded with a per-row
//    chunk swizzle (swz_col for K, swz_tr for V).
//  * Lazy rescale: the running max only moves when a row's max grows by more
//    than 2^8, so O is rescaled rarely; P <= 2^8 stays exact in fp16/bf16 and
//    the final O / l and LSE use the same max, so results are unchanged.
//  * Only tiles that straddle a mask edge or the KV tail evaluate the mask per
//    element; fully masked blocks of such tiles run the same instructions
//    with P = 0 (one straight path keeps the accumulators in place).
//  * Block-sparse maps: the workgroup walks only the KV tiles whose
//    128 x 128 block is computed for some of its rows (a list built in LDS
//    at the start); in a listed tile, a wave whose own block is removed
//    skips the softmax and feeds P = 0 to its PV MFMAs (a branch around the
//    MFMA phase costs the ping-pong loop its register budget); the 4-wave
//    form (D = 256) skips the whole tile for that wave.
#include "flexatt_device.h"
#include "flexatt_kernels.h"

#ifndef FLEXATT_D
#error "FLEXATT_D (head dim) must be defined"
#endif

namespace flexatt {

template <int D>
struct FwdCfg {
  static constexpr int NW = D <= 128 ? 8 : 4;   // waves per workgroup
  // waves per SIMD the register budget targets: at D = 64 two workgroups
  // share a CU (64 KB of LDS each), whose VALU-heavy phases then overlap
  // (D = 32 would spill at that budget)
  static constexpr int WPE = D == 64 ? 4 : (D <= 128 ? 2 : 1);
#ifdef FLEXATT_FWD_BN
  static constexpr int BN = FLEXATT_FWD_BN;  // tuning override
#else
  static constexpr int BN = D == 32 ? 128 : (D == 256 ? 32 : 64);  // KV rows per tile
#endif
  static constexpr int NB = BN / 32;
  static constexpr int KC = D / 16;
  static constexpr int DB = D / 32;
  static constexpr int CPR = D / 8;         // 16-byte chunks per row
  static constexpr int ROWB = D * 2;        // bytes per tile row
  static constexpr int TILEB = BN * ROWB;   // bytes per tile of one tensor
  static constexpr int E = TILEB / (1024 * NW);  // 1 KB loads per wave per tensor per tile
  // Ping-pong schedule (two waves per SIMD, one phase apart) when the
  // workgroup has 8 waves; 4-wave workgroups (D = 256) run one wave per SIMD.
  static constexpr bool PP = NW == 8;
  static constexpr int STAGES = PP ? 4 : 3;
#ifdef FLEXATT_FWD_PF
  static constexpr int PF = FLEXATT_FWD_PF;  // tuning override
#else
  static constexpr int PF = 2;  // MFMA pairs whose LDS reads are issued ahead
#endif
  static_assert(E >= 1 && E * 1024 * NW == TILEB, "tile must split into 1 KB loads per wave");
};

constexpr float kRescaleThreshold = 8.0f;  // log2 units

template <class T, int D, bool SOFTCAP, bool ALIBI, bool BLK>
__global__ __launch_bounds__(FwdCfg<D>::NW * 64) __attribute__((amdgpu_waves_per_eu(FwdCfg<D>::WPE, FwdCfg<D>::WPE)))
void fwd_mfma_kernel(FwdArgs a) {
  using C = FwdCfg<D>;
  using M = Mfma<T>;
  using V8 = typename M::v8;
  __shared__ __attribute__((aligned(1024))) char smem[C::STAGES * 2 * C::TILEB];

  const Shape& p = a.p;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar branches)
  const int h = lane >> 5, l32 = lane & 31;

  // Work item: (b, hkv, head group, q-tile); the longest causal tiles first.
  const int gp = a.gpack;
  const int bmh = 32 * (C::NW / gp);  // query rows per head
  const int ngs = p.G / gp;
  int kq, rest;  // kq = 0: the last query tile, the longest causal band
  if (!xcd_lpt_item(blockIdx.x, a.nqt, ngs * p.B * p.Hkv, kq, rest)) {
    const int w = xcd_remap(blockIdx.x, gridDim.x);
    kq = w % a.nqt;
    rest = w / a.nqt;
  }
  const int qt = a.nqt - 1 - kq;
  const int gs = rest % ngs;
  rest /= ngs;
  const int hk = rest % p.Hkv, b = rest / p.Hkv;
  const int hq = hk * p.G + gs * gp + wave % gp;
  const int m0 = qt * bmh;
  const int mw = m0 + 32 * (wave / gp);
  const int my_m = mw + l32;

  const T* qp = (const T*)a.q.data + b * a.q.sb + hq * a.q.sh;
  const T* kp = (const T*)a.k.data + b * a.k.sb + hk * a.k.sh;
  const T* vp = (const T*)a.v.data + b * a.v.sb + hk * a.v.sh;

  // Q rows past Sq load row Sq - 1 (finite scores; their O and LSE are not
  // stored).  Nothing reads qf before the first tile copies are issued, so
  // the Q loads and the copies share one memory round trip.
  V8 qf[C::KC];
  {
    const int r = min(my_m, p.Sq - 1);
    const T* src = qp + (int64_t)r * a.q.ss + 8 * h;
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc) qf[kc] = as_v8<V8>(ld_global16(src + 16 * kc));
  }

  int kv_lo = 0, kv_hi = p.Skv;
  if (p.causal) kv_hi = min(kv_hi, m0 + bmh);
  if (p.window > 0) kv_lo = max(0, m0 - p.window);
  // document masks: this lane's bounds and the KV range of the workgroup's rows
  int dlo, dhi;
  doc_bounds(p, b, min(my_m, p.Sq - 1), dlo, dhi);
  if (p.doc) {
    int l0, h0, l1, h1;
    doc_bounds(p, b, min(m0, p.Sq - 1), l0, h0);
    doc_bounds(p, b, min(m0 + bmh, p.Sq) - 1, l1, h1);
    kv_lo = max(kv_lo, l0);
    kv_hi = min(kv_hi, h1);
  }
  const int t_lo = kv_lo / C::BN;
  const int t_hi = (kv_hi + C::BN - 1) / C::BN;
  // This lane's row attends to the keys [row_lo, row_lo + row_w): causal,
  // window, KV tail and document bounds as one interval, so that a masked
  // tile tests each element with one unsigned compare against its offset.
  int row_lo = max(dlo, 0), row_hi = min(dhi, p.Skv);
  if (p.causal) row_hi = min(row_hi, my_m + 1);
  if (p.window > 0) row_lo = max(row_lo, my_m - p.window);
  const unsigned row_w = (unsigned)max(row_hi - row_lo, 0);

  // Block-sparse mask: this wave's row of the block map over the
  // workgroup's KV range, kept in (dynamic) LDS so that the tile loop issues
  // no memory operation besides its tile copies; then the list of the tiles
  // whose block is computed for some row of the workgroup.  The tile loop
  // walks that list (v = 0 .. nv-1 -> tile tile_of(v)); removed tiles are
  // neither copied nor computed.  Without a map the list is [t_lo, t_hi).
  extern __shared__ unsigned char sblk[];
  __shared__ int s_nv;
  const int bstride = a.bstride;
  unsigned short* tlist = (unsigned short*)(sblk + C::NW * bstride);
  const int kb_base = t_lo * C::BN / kBlk;
  int nv = t_hi - t_lo;
  if (BLK && t_lo < t_hi) {
    const unsigned char* row = block_row(p, b, hq, min(mw, p.Sq - 1));
    const int nkb = (t_hi * C::BN - 1) / kBlk - kb_base + 1;
    for (int i = lane; i < nkb; i += 64) sblk[wave * bstride + i] = row[kb_base + i];
    __syncthreads();
    if (wave == 0) {
      int base = 0;
      for (int t0 = t_lo; t0 < t_hi; t0 += 64) {
        const int t = t0 + lane;
        bool live = false;
        if (t < t_hi) {
          const int kb = t * C::BN / kBlk - kb_base;
#pragma unroll
          for (int w = 0; w < C::NW; ++w) live = live || sblk[w * bstride + kb] != 0;
        }
        const unsigned long long m = __builtin_amdgcn_ballot_w64(live);
        if (live) tlist[base + __builtin_popcountll(m & ((1ull << lane) - 1))] = (unsigned short)(t - t_lo);
        base += __builtin_popcountll(m);
      }
      if (lane == 0) s_nv = base;
    }
    __syncthreads();
    nv = __builtin_amdgcn_readfirstlane(s_nv);
  }
  auto tile_of = [&](int v) -> int {
    if constexpr (BLK) return t_lo + __builtin_amdgcn_readfirstlane((int)tlist[v]);
    else return t_lo + v;
  };
  // whether the 128 x 128 block of this wave's rows and KV row n0 is computed
  auto block_live = [&](int n0) { return !BLK || sblk[wave * bstride + n0 / kBlk - kb_base] != 0; };

  // Direct global -> LDS copy of tile t into stage st: E 1 KB loads per
  // tensor per wave; lane l of load e covers physical chunk q of the tile.
  const unsigned lds0 = lds_addr_of(smem);
  auto issue = [&](int t, int st) {
    const int n0 = t * C::BN;
    const unsigned sbase = lds0 + st * 2 * C::TILEB;
#pragma unroll
    for (int e = 0; e < C::E; ++e) {
      const int blk = wave * C::E + e;
      const int q = blk * 64 + lane;
      const int row = q / C::CPR, pc = q % C::CPR;
      const int64_t n = min(n0 + row, p.Skv - 1);
      load_lds16(kp + n * a.k.ss + swz_col<C::CPR>(row, pc) * 8, sbase + blk * 1024);
      load_lds16(vp + n * a.v.ss + swz_tr_inv<C::CPR>(row, pc) * 8, sbase + C::TILEB + blk * 1024);
    }
  };

  // Lane-constant byte offsets of this lane's LDS reads inside a tile.
  int koff[C::KC], voff[C::DB];
  const int tr_row = 4 * h + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
  for (int kc = 0; kc < C::KC; ++kc) koff[kc] = l32 * C::ROWB + swz_col<C::CPR>(l32, 2 * kc + h) * 16;
#pragma unroll
  for (int db = 0; db < C::DB; ++db)
    voff[db] = tr_row * C::ROWB + swz_tr<C::CPR>(tr_row, 4 * db + (tr_col >> 3)) * 16 + (tr_col & 7) * 2;

  f32x16 acc[C::DB];
#pragma unroll
  for (int db = 0; db < C::DB; ++db) acc[db] = f32x16{};
  float m_run = kNegInf, l_run = 0.f;
  const float slope_log2 = ALIBI ? p.alibi[hq] * kLog2e : 0.f;

  // Raw-score fast path (no soft-cap, no ALiBi): scores stay unscaled and
  // the scale is folded into the exp2 FMA.  A negative scale is moved into
  // the sign of Q (exact), a zero scale replaced by a tiny one, so that the
  // row max is always a max and masked scores (-inf) map to exp2(-inf) = 0.
  constexpr bool RAW = !SOFTCAP && !ALIBI;
  float c2 = p.scale_log2;
  if constexpr (RAW) {
    if (c2 < 0.f) {
#pragma unroll
      for (int kc = 0; kc < C::KC; ++kc)
        qf[kc] = as_v8<V8>(__builtin_bit_cast(i32x4, qf[kc]) ^ i32x4{(int)0x80008000, (int)0x80008000,
                                                                     (int)0x80008000, (int)0x80008000});
      c2 = -c2;
    }
    if (c2 == 0.f) c2 = 1e-30f;
  }

  auto tile_body = [&](const char* sK, const char* sV, int n0, bool need_mask) {
    // S^T for every 32-row block of the tile.
    f32x16 s[C::NB];
#pragma unroll
    for (int bb = 0; bb < C::NB; ++bb) {
      s[bb] = f32x16{};
#pragma unroll
      for (int kc = 0; kc < C::KC; ++kc)
        s[bb] = M::mma(as_v8<V8>(lds_read16(sK + bb * 32 * C::ROWB + koff[kc])), qf[kc], s[bb]);
    }
    // keep the K reads a few ahead of the MFMAs that consume them
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < C::NB * C::KC - 4; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);

    // scores -> log2 domain (transform paths), mask (edge tiles only)
    if constexpr (!RAW) {
      const float fb = (float)(my_m - n0 - 4 * h);  // i - j = fb - (32 bb + 8 (r / 4) + r % 4)
#pragma unroll
      for (int bb = 0; bb < C::NB; ++bb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float tv;
          s[bb][r] = score_log2_d<SOFTCAP, ALIBI>(s[bb][r], p, slope_log2,
                                                 fb - (float)(32 * bb + 8 * (r >> 2) + (r & 3)), tv);
        }
    }
    if (need_mask) {  // (removed blocks never get here)
      const int a0 = row_lo - n0 - 4 * h;  // element offset of the interval's start
#pragma unroll
      for (int bb = 0; bb < C::NB; ++bb)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if ((unsigned)(32 * bb + 8 * (r >> 2) + (r & 3) - a0) >= row_w) s[bb][r] = kNegInf;
    }

    // tile row max (pairwise tree), exchanged between the wave halves
    float mx;
    {
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = fmaxf(s[0][2 * i], s[0][2 * i + 1]);
#pragma unroll
      for (int bb = 1; bb < C::NB; ++bb)
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = fmaxf(v[i], fmaxf(s[bb][2 * i], s[bb][2 * i + 1]));
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = fmaxf(v[i], v[i + 4]);
      mx = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
    }
    if constexpr (RAW) mx *= c2;
    mx = fmaxf(mx, swap_halves(mx));
    if (mx != mx) mx = kNegInf;
    const bool grow = mx > m_run + kRescaleThreshold;
    if (__builtin_amdgcn_ballot_w64(grow)) {
      const float m_new = grow ? mx : m_run;
      const float alpha = grow ? fast_exp2(m_run - m_new) : 1.f;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < C::DB; ++db) scale_inplace(acc[db], alpha);
      m_run = m_new;
    }
    const float m_use = (m_run == kNegInf) ? 0.f : m_run;

    // P = exp2(y - m), row sums, O^T += V^T P^T
    float rs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int bb = 0; bb < C::NB; ++bb) {
      f32x16 e;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if constexpr (RAW) e[r] = fast_exp2(__builtin_fmaf(s[bb][r], c2, -m_use));
        else e[r] = fast_exp2(s[bb][r] - m_use);
        rs[r & 3] += e[r];
      }
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const V8 pb = pack8<T>(e, 8 * c);
        const char* vr = sV + (32 * bb + 16 * c) * C::ROWB;
#pragma unroll
        for (int db = 0; db < C::DB; ++db) {
          const i16x4 lo = lds_read_tr4(vr + voff[db]);
          const i16x4 hi = lds_read_tr4(vr + 8 * C::ROWB + voff[db]);
          acc[db] = M::mma(cat_tr<V8>(lo, hi), pb, acc[db]);
        }
      }
    }
    l_run += (rs[0] + rs[1]) + (rs[2] + rs[3]);
    // block 0's exps first, then each PV MFMA of block bb paired with
    // transpose reads and a share of block bb+1's exp/convert VALU work
    __builtin_amdgcn_sched_group_barrier(0x002, 24, 1);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 1);
#pragma unroll
    for (int i = 0; i < 2 * C::DB * C::NB; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 1);
    }
  };

  if constexpr (C::PP) {
    // Ping-pong.  Waves 0-3 and 4-7 (one of each on every SIMD) run the same
    // program one phase apart, phases separated by workgroup barriers:
    //   MFMA phase  M(t): S^T(t) = K(t) Q^T and O^T += V^T P(t-1)^T, 32
    //                     independent MFMAs fed from LDS, plus the copies of
    //                     tile t+2;
    //   VALU phase  V(t): mask, row max, rescale, P(t) = exp2(y - m), its row
    //                     sums and its packing into PV operands.
    // While one wave of a SIMD is in its MFMA phase the other is in its VALU
    // phase.  (Moving the packing and row sums into the MFMA phase, or the
    // copies into the VALU phase, measured slower: the two phases are about
    // equally long.)
    // The v-th tile of the walk lives in stage v % 4 from its copy (issued at
    // the start of M(v-2)) until B's M(v+1) has read its V; the copy of tile
    // v+4 into that stage is issued at M(v+2), after the barrier that ends
    // B's M(v+1).
    const int grp = wave >> 2;
    // Tile copies are issued in walk order, one per M phase, past the last
    // tile as redundant copies of it into a free stage, so that each wave
    // always has exactly one copy in flight beyond the tile it needs next and
    // every wait is vmcnt(2E) (vector memory operations complete in order, a
    // tile is 2E of them per wave).
    int64_t koffs[C::E], voffs[C::E];  // byte offsets of this lane's chunks within a tile
#pragma unroll
    for (int e = 0; e < C::E; ++e) {
      const int q = (wave * C::E + e) * 64 + lane;
      const int row = q / C::CPR, pc = q % C::CPR;
      koffs[e] = ((int64_t)row * a.k.ss + swz_col<C::CPR>(row, pc) * 8) * (int64_t)sizeof(T);
      voffs[e] = ((int64_t)row * a.v.ss + swz_tr_inv<C::CPR>(row, pc) * 8) * (int64_t)sizeof(T);
    }
    const int64_t kstep = (int64_t)C::BN * a.k.ss * (int64_t)sizeof(T);
    const int64_t vstep = (int64_t)C::BN * a.v.ss * (int64_t)sizeof(T);
    // copy cursors: stepped tile by tile without a map, set from the list with one
    const char* kcur = (const char*)(kp + (int64_t)t_lo * C::BN * a.k.ss);
    const char* vcur = (const char*)(vp + (int64_t)t_lo * C::BN * a.v.ss);
    int next_v = 0;
    auto issue_next = [&]() {
      const int v = next_v++;
      const int st = v & 3;
      int t = t_lo + v;
      if constexpr (BLK) {
        t = tile_of(min(v, nv - 1));
        kcur = (const char*)kp + t * kstep;
        vcur = (const char*)vp + t * vstep;
      }
      if (v < nv && (t + 1) * C::BN <= p.Skv) {
        const unsigned dst = lds0 + st * 2 * C::TILEB + wave * C::E * 1024;
#pragma unroll
        for (int e = 0; e < C::E; ++e) {
          load_lds16(kcur + koffs[e], dst + e * 1024);
          load_lds16(vcur + voffs[e], dst + e * 1024 + C::TILEB);
        }
        kcur += kstep;
        vcur += vstep;
      } else {
        // KV tail (rows clamped to Skv - 1) or a redundant copy of the last tile
        issue(BLK ? t : min(t, t_hi - 1), st);
      }
    };
    auto wait_tile = [&]() { wait_vmcnt<2 * C::E>(); };
    f32x16 s[C::NB];  // scores of the tile in flight
    V8 P[2 * C::NB];  // exp2(y - m) of the previous tile as the PV MFMA operand

    // Tiles [tm_lo, tm_hi) are fully allowed for every row of this wave:
    // below tm_lo a row may be outside the window, from tm_hi on a tile may
    // cross the causal diagonal or the KV tail.
    int tm_hi = p.Skv / C::BN;  // tiles wholly inside the KV length
    if (p.causal) tm_hi = min(tm_hi, (mw + 1) / C::BN);  // n0 + BN - 1 <= mw
    int tm_lo = 0;
    if (p.window > 0) tm_lo = max(0, (mw + 31 - p.window + C::BN - 1) / C::BN);  // mw + 31 - n0 <= window
    if (p.doc) {  // full tiles lie inside the key interval of every row of the wave:
      int l0, h0, l1, h1;  // [lo of its last row, hi of its first row) (bounds are non-decreasing)
      doc_bounds(p, b, min(mw, p.Sq - 1), l0, h0);
      doc_bounds(p, b, min(mw + 31, p.Sq - 1), l1, h1);
      tm_lo = max(tm_lo, (l1 + C::BN - 1) / C::BN);
      tm_hi = min(tm_hi, h0 / C::BN);
      if (tm_hi < tm_lo) tm_hi = tm_lo;
    }
    tm_hi = __builtin_amdgcn_readfirstlane(tm_hi);
    tm_lo = __builtin_amdgcn_readfirstlane(tm_lo);
    auto softmax = [&](int n0) {
      if (!block_live(n0)) {  // a removed block: P = 0 for the PV MFMAs, if they run
#pragma unroll
        for (int i = 0; i < 2 * C::NB; ++i) P[i] = V8{};
        return;
      }
      if constexpr (!RAW) {
        // i - j = fb - (32 bb + 8 (r / 4) + r % 4), exact in fp32
        const float fb = (float)(my_m - n0 - 4 * h);
#pragma unroll
        for (int bb = 0; bb < C::NB; ++bb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            float tv;
            s[bb][r] = score_log2_d<SOFTCAP, ALIBI>(s[bb][r], p, slope_log2,
                                                   fb - (float)(32 * bb + 8 * (r >> 2) + (r & 3)), tv);
          }
      }
      const int tn = n0 / C::BN;
      if (tn < tm_lo || tn >= tm_hi) {
        // element (bb, r) is key n0 + 32 bb + 8 (r / 4) + 4 h + r % 4
        const int a0 = row_lo - n0 - 4 * h;
#pragma unroll
        for (int bb = 0; bb < C::NB; ++bb) {
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if ((unsigned)(32 * bb + 8 * (r >> 2) + (r & 3) - a0) >= row_w) s[bb][r] = kNegInf;
          pin(s[bb]);  // finished inside the branch (no selects after it)
        }
      }
      float mp[2 * C::NB];
#pragma unroll
      for (int bb = 0; bb < C::NB; ++bb) max16_partial(s[bb], mp[2 * bb], mp[2 * bb + 1]);
      float mx;
      if constexpr (C::NB == 1) mx = max2(mp[0], mp[1]);
      else if constexpr (C::NB == 2) mx = max2(max3(mp[0], mp[1], mp[2]), mp[3]);
      else {
        float u = max3(mp[0], mp[1], mp[2]);
        u = max3(u, mp[3], mp[4]);
        u = max3(u, mp[5], mp[6]);
        mx = max2(u, mp[7]);
      }
      if constexpr (RAW) mx *= c2;
      mx = fmaxf(mx, swap_halves(mx));
      if (mx != mx) mx = kNegInf;
      const bool grow = mx > m_run + kRescaleThreshold;
      if (__builtin_amdgcn_ballot_w64(grow)) {
        const float m_new = grow ? mx : m_run;
        const float alpha = grow ? fast_exp2(m_run - m_new) : 1.f;
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < C::DB; ++db) scale_inplace(acc[db], alpha);
        m_run = m_new;
      }
      const float m_use = (m_run == kNegInf) ? 0.f : m_run;
      // (fp32 adds for the row sums: dot2 instructions share the matrix pipe
      // and would stall behind the other wave's MFMAs)
      float rs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int bb = 0; bb < C::NB; ++bb) {
        f32x16 e;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          if constexpr (RAW) e[r] = fast_exp2(__builtin_fmaf(s[bb][r], c2, -m_use));
          else e[r] = fast_exp2(s[bb][r] - m_use);
          rs[r & 3] += e[r];
        }
        P[2 * bb] = pack8<T>(e, 0);
        P[2 * bb + 1] = pack8<T>(e, 8);
      }
      l_run += (rs[0] + rs[1]) + (rs[2] + rs[3]);
      // done before the barrier
#pragma unroll
      for (int i = 0; i < 2 * C::NB; ++i) pin(P[i]);
      pin(l_run);
    };
    // phase inputs are read only after the barrier that ends their producer
    auto pin_s = [&]() {
#pragma unroll
      for (int bb = 0; bb < C::NB; ++bb) pin(s[bb]);
    };
    auto pin_p = [&]() {
#pragma unroll
      for (int i = 0; i < 2 * C::NB; ++i) pin(P[i]);
    };

    // MFMA phase: PV of the previous tile (stage sv) and/or S^T of the next
    // (stage sk), interleaved so that the two accumulator sets never wait on
    // each other; LDS reads are kept PF MFMA pairs ahead.
    constexpr int NPV = 2 * C::NB * C::DB;  // == NB * KC
    auto mphase = [&](int sv, int sk, bool do_pv, bool do_s) {
      const char* sV = smem + sv * 2 * C::TILEB + C::TILEB;
      const char* sK = smem + sk * 2 * C::TILEB;
      if (do_s) {
#pragma unroll
        for (int bb = 0; bb < C::NB; ++bb) s[bb] = f32x16{};
      }
#pragma unroll
      for (int i = 0; i < NPV; ++i) {
        if (do_pv) {
          const int db = i % C::DB, c = (i / C::DB) & 1, bb = i / (2 * C::DB);
          const char* vr = sV + (32 * bb + 16 * c) * C::ROWB + voff[db];
          const i16x4 lo = lds_read_tr4(vr);
          const i16x4 hi = lds_read_tr4(vr + 8 * C::ROWB);
          acc[db] = M::mma(cat_tr<V8>(lo, hi), P[2 * bb + c], acc[db]);
        }
        if (do_s) {
          const int bb = i % C::NB, kc = i / C::NB;
          s[bb] = M::mma(as_v8<V8>(lds_read16(sK + bb * 32 * C::ROWB + koff[kc])), qf[kc], s[bb]);
        }
      }
      if (do_pv && do_s) {
        __builtin_amdgcn_sched_group_barrier(0x100, 3 * C::PF, 2);
#pragma unroll
        for (int i = 0; i < NPV - C::PF; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 2);
          __builtin_amdgcn_sched_group_barrier(0x100, 3, 2);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * C::PF, 2);
      }
    };

    if (nv > 0) {
      issue_next();  // v = 0
      issue_next();  // v = 1
      wait_tile();
      __syncthreads();
      if (grp) __syncthreads();  // second half starts one phase late
      issue_next();  // v = 2
      mphase(0, 0, false, true);
      wait_tile();
      __syncthreads();
      pin_s();
      for (int v = 0; v + 1 < nv; ++v) {
        softmax(tile_of(v) * C::BN);
        wait_tile();
        __syncthreads();
        pin_p();
        // the MFMA phase issues ahead of the other wave's softmax on the SIMD
        // (measured 1-1.5% faster; raising the softmax wave instead is slower)
        __builtin_amdgcn_s_setprio(1);
        issue_next();  // v + 3
        mphase(v & 3, (v + 1) & 3, true, true);
        __builtin_amdgcn_s_setprio(0);
        wait_tile();
        __syncthreads();
        pin_s();
      }
      softmax(tile_of(nv - 1) * C::BN);
      wait_tile();
      __syncthreads();
      pin_p();
      mphase((nv - 1) & 3, 0, true, false);
      wait_vmcnt<0>();  // no copy may land after the workgroup's LDS is released
      __syncthreads();
      if (!grp) __syncthreads();  // first half: match the second's count
    }
  } else {
    if (nv > 0) issue(tile_of(0), 0);
    if (nv > 1) issue(tile_of(1), 1);
    int st = 0;
    for (int v = 0; v < nv; ++v) {
      if (v + 1 < nv) wait_vmcnt<2 * C::E>();
      else wait_vmcnt<0>();
      __syncthreads();
      if (v + 2 < nv) issue(tile_of(v + 2), st == 0 ? 2 : st - 1);
      const char* sK = smem + st * 2 * C::TILEB;
      const char* sV = sK + C::TILEB;
      const int n0 = tile_of(v) * C::BN;
      // Per element masking only on tiles that cut the causal diagonal, the
      // window edge or the KV tail for some row of this wave.
      const bool need_mask = (n0 + C::BN > p.Skv) || (p.causal && n0 + C::BN - 1 > mw) ||
                             (p.window > 0 && mw + 31 - n0 > p.window) || p.doc || !block_live(n0);
      if (block_live(n0)) tile_body(sK, sV, n0, need_mask);  // removed blocks are skipped
      st = st == 2 ? 0 : st + 1;
    }
  }

  const float l_tot = l_run + swap_halves(l_run);
  const bool empty = !(l_tot > 0.f);
  const float inv = empty ? 0.f : 1.0f / l_tot;
  // O leaves through LDS: each lane holds 4 columns of one row, which would
  // make every store instruction touch 32 rows; staged as the wave's 32 x D
  // row-major tile (16-byte chunk c of row r at c ^ (r % CPR)), it is stored
  // 16 contiguous bytes per lane, 64 / CPR whole rows per instruction.
  if constexpr (!C::PP) __syncthreads();  // the last tile's LDS reads are done
  char* so = smem + wave * 32 * C::ROWB;
#pragma unroll
  for (int db = 0; db < C::DB; ++db) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = 4 * db + i;  // columns 32 db + 8 i .. + 7; this lane's half at byte 8 h
      *(i32x2*)(so + l32 * C::ROWB + (c ^ (l32 % C::CPR)) * 16 + 8 * h) =
          pack4<T>(acc[db][4 * i] * inv, acc[db][4 * i + 1] * inv, acc[db][4 * i + 2] * inv, acc[db][4 * i + 3] * inv);
    }
  }
  {
    constexpr int RPI = 64 / C::CPR;  // rows per store instruction
    const int cc = lane % C::CPR;
    T* ob = (T*)a.o.data + b * a.o.sb + hq * a.o.sh + cc * 8;
#pragma unroll
    for (int k = 0; k < 32 / RPI; ++k) {
      const int rr = k * RPI + lane / C::CPR;
      const i32x4 x = lds_read16(so + rr * C::ROWB + (cc ^ (rr % C::CPR)) * 16);
      if (mw + rr < p.Sq) *(i32x4*)(ob + (int64_t)(mw + rr) * a.o.ss) = x;
    }
  }
  if (my_m < p.Sq && h == 0)
    a.lse[(int64_t)(b * p.Hq + hq) * p.Sq + my_m] = empty ? kNegInf : (m_run + log2f(l_tot)) * kLn2;
}

// Heads per workgroup: the largest power of two that divides G, capped at NW.
inline int gqa_pack(int G, int nw) {
  const int gp = G & (-G);
  return gp < nw ? gp : nw;
}

template <class T, int D>
hipError_t launch_fwd_mfma(const FwdArgs& a, hipStream_t st) {
  using C = FwdCfg<D>;
#ifndef FLEXATT_FWD_WS
#define FLEXATT_FWD_WS 1  // tuning override: 0 keeps D = 256 on the 4-wave form
#endif
  // D = 256: the wave-specialised pairs of fwd_ws.hip (block maps whose
  // lists do not fit beside its 145 KB of LDS stay here)
  if constexpr (D == 256 && FLEXATT_FWD_WS) {
    if (fwd_ws_fits(a.p)) return std::is_same<T, __bf16>::value ? fwd_ws_bf16_d256(a, st) : fwd_ws_f16_d256(a, st);
  }
  FwdArgs x = a;
  x.gpack = gqa_pack(a.p.G, C::NW);
  const int bmh = 32 * (C::NW / x.gpack);
  x.nqt = (a.p.Sq + bmh - 1) / bmh;
  const dim3 grid(x.nqt * (a.p.G / x.gpack) * a.p.B * a.p.Hkv), block(C::NW * 64);
  const bool sc = a.p.cap > 0.f, al = a.p.alibi != nullptr;
  // block-sparse maps: each wave's block-map row, then the workgroup's tile list
  x.bstride = (a.p.blk_nk + 3) & ~3;
  const int tiles = (a.p.Skv + C::BN - 1) / C::BN;
  const size_t dyn = a.p.blk ? (size_t)C::NW * x.bstride + 2 * (size_t)(tiles + 2) : 0;
  if (a.p.blk) {
    if (sc && al) hipLaunchKernelGGL((fwd_mfma_kernel<T, D, true, true, true>), grid, block, dyn, st, x);
    else if (sc) hipLaunchKernelGGL((fwd_mfma_kernel<T, D, true, false, true>), grid, block, dyn, st, x);
    else if (al) hipLaunchKernelGGL((fwd_mfma_kernel<T, D, false, true, true>), grid, block, dyn, st, x);
    else hipLaunchKernelGGL((fwd_mfma_kernel<T, D, false, false, true>), grid, block, dyn, st, x);
  } else {
    if (sc && al) hipLaunchKernelGGL((fwd_mfma_kernel<T, D, true, true, false>), grid, block, 0, st, x);
    else if (sc) hipLaunchKernelGGL((fwd_mfma_kernel<T, D, true, false, false>), grid, block, 0, st, x);
    else if (al) hipLaunchKernelGGL((fwd_mfma_kernel<T, D, false, true, false>), grid, block, 0, st, x);
    else hipLaunchKernelGGL((fwd_mfma_kernel<T, D, false, false, false>), grid, block, 0, st, x);
  }
  return hipGetLastError();
}

#define FLEXATT_CAT2(a, b) a##b
#define FLEXATT_CAT(a, b) FLEXATT_CAT2(a, b)
hipError_t FLEXATT_CAT(fwd_mfma_bf16_d, FLEXATT_D)(const FwdArgs& a, hipStream_t st) {
  return launch_fwd_mfma<__bf16, FLEXATT_D>(a, st);
}
hipError_t FLEXATT_CAT(fwd_mfma_f16_d, FLEXATT_D)(const FwdArgs& a, hipStream_t st) {
  return launch_fwd_mfma<_Float16, FLEXATT_D>(a, st);
}

}  // namespace flexatt
