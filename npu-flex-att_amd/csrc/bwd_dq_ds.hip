// Flash-attention backward dQ from the staged dS (fp16/bf16, D = 64, 128 or 256, gfx950).
//
// Semantics: the dQ GEMM of npu_flash_attention.py:399 (dq += ds . k, ds
// rounded to the input dtype before tl.dot), dQ = scale * dS K, with dS as
// the dK/dV kernel (bwd_kv.hip) formed and stored it: P (dP - Delta)
// (1 - tanh^2), masked, rounded to the input dtype, without the scale.  The
// dK/dV kernel already recomputed S and dP for every attended pair, so this
// kernel only streams dS and K: one GEMM of the five, where a dQ kernel that
// recomputes runs three.
//
// Decomposition
//  * A workgroup is 4 waves, one per SIMD, for one (b, KV head) and 16 query
//    slots, or at D = 256 8 waves, two per SIMD, and 8 slots (a slot is 32
//    rows of one query head): nh heads (4, 2 or 1, the largest dividing
//    Hq / Hkv) x slots / nh query tiles.  Wave v owns slots NSL v ..
//    NSL v + NSL - 1 (NSL = 4, or 1 at D = 256), lane = query row; its dQ^T
//    (NSL slots x D x 32 fp32) lives in the accumulation registers.
//  * The workgroup walks the 64-row KV sub-blocks its slots' dS bands cover.
//    K rows (16 KB per sub-block, read by all waves) go global -> LDS with
//    direct-to-LDS loads three sub-blocks ahead into four stages; dS goes
//    global -> registers two sub-blocks ahead, already in the MFMA B operand
//    layout the dK/dV kernel stored it in (64 KB per sub-block and CU, read
//    once, so 128 KB in flight per CU).
//  * Per sub-block and wave: KS x DB x NSL MFMAs dQ^T += K^T dS^T; each K^T
//    operand (two LDS transpose reads) feeds the wave's slots.
//  * A slot whose band does not cover a sub-block skips its MFMAs and loads
//    a valid address instead, so every wave issues the same memory
//    operations per sub-block and fixed vmcnt waits hold.
// HBM-bound: dS is read once (2 bytes per attended pair per query head).
// Deterministic: every output element is owned by one lane and accumulated in
// a fixed order.
#include "flexatt_device.h"
#include "flexatt_kernels.h"

#ifndef FLEXATT_D
#error "FLEXATT_D (head dim) must be defined"
#endif

namespace flexatt {

#if FLEXATT_D == 128 || FLEXATT_D == 64 || FLEXATT_D == 256

#ifndef FLEXATT_DQ_W256
#define FLEXATT_DQ_W256 8  // tuning override: 4 waves (one per SIMD, two slots each) at D = 256
#endif
template <int D>
struct DqsCfg {
  // waves per workgroup: one per SIMD (D = 64, 128); at D = 256 two per SIMD
  // with one slot each (128 accumulators), so that one wave's loads and LDS
  // reads overlap the other's MFMAs
  static constexpr int NW = D == 256 ? FLEXATT_DQ_W256 : 4;
  static constexpr int WPE = NW / 4;            // waves per SIMD
  static constexpr int NSL = D == 256 ? 8 / NW : 4;  // query slots per wave (256 accumulators per SIMD at D = 256)
  static constexpr int SLOTS = NW * NSL;        // query slots per workgroup
  static constexpr int SB = 64;                // KV rows per sub-block
  static constexpr int KS = SB / 16;           // k steps per sub-block
  static constexpr int DB = D / 32;            // d-blocks of dQ^T
  static constexpr int CPR = D / 8;            // 16-byte chunks per K row
  static constexpr int ROWB = 2 * D;           // bytes per K row
  static constexpr int KTILEB = SB * ROWB;     // K rows of a sub-block
  static constexpr int EK = KTILEB / (1024 * NW);  // 1 KB K copies per wave
  static constexpr int SUBB = kDsUnitB * SB / kDsKB;  // one slot's dS of a sub-block
  static constexpr int KSTAGES = 4;
  static constexpr int KAHEAD = KSTAGES - 1;   // K copies run this many sub-blocks ahead
  static constexpr int DAHEAD = 2;             // dS loads run this many sub-blocks ahead
  static constexpr int NDS = NSL * KS;         // dS operands (1 KB loads) per sub-block
  static_assert(EK * 1024 * NW == KTILEB && SUBB == KS * 1024, "1 KB pieces");
  static_assert(KSTAGES * KTILEB <= 128 * 1024, "LDS");
};

template <class T, int D, bool BLK>
__global__ __launch_bounds__(DqsCfg<D>::NW * 64) __attribute__((amdgpu_waves_per_eu(DqsCfg<D>::WPE, DqsCfg<D>::WPE)))
void bwd_dq_ds_kernel(BwdArgs a) {
  using C = DqsCfg<D>;
  using M = Mfma<T>;
  using V8 = typename M::v8;
  static_assert((D == 64 || D == 128 || D == 256) && C::KS == 4, "the MFMA blocking assumes 64-row sub-blocks");
  __shared__ __attribute__((aligned(1024))) char smem[C::KSTAGES * C::KTILEB];

  const Shape& p = a.p;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31;

  // Work item: (b, hkv, head group, query block), the query blocks of one
  // (b, hkv) consecutive (they share K in one XCD's L2), longest causal
  // bands first.  A block holds SLOTS slots: nh heads x (SLOTS / nh) query tiles.
  const int nh = a.ntiles & 0xff;  // heads per workgroup: 4, 2 or 1 (divides G)
  const int nqb = a.ntiles >> 8;   // query blocks per head group
  const int nq = C::SLOTS / nh;    // query tiles per block
  const int ngs = p.G / nh;
  const int slot = queue_slot(a.queue, a.nstatic);
  if (slot >= (int)gridDim.x) return;  // (a counter that was not cleared)
  int kq, rest;  // kq = 0: the last query block, the longest causal band
  if (!xcd_lpt_item(slot, nqb, ngs * p.B * p.Hkv, kq, rest)) {
    const int w = xcd_remap(slot, gridDim.x);
    kq = w % nqb;
    rest = w / nqb;
  }
  const int qb = nqb - 1 - kq;
  const int hg = rest % ngs;
  rest /= ngs;
  const int hk = rest % p.Hkv, b = rest / p.Hkv;

  const int nqt = (p.Sq + kDsQT - 1) / kDsQT;
  const int nkb = (p.Skv + kDsKB - 1) / kDsKB;
  const int nsb = (p.Skv + C::SB - 1) / C::SB;  // sub-blocks holding key rows
  constexpr int SPU = kDsKB / C::SB;            // sub-blocks per dS unit
  // Slot c of wave v: 16 slots ordered (tile, head) so that the four slots
  // of a wave lie in one aligned group of four query tiles (one causal band
  // end).
  auto slot_of = [&](int v, int c, int& hq, int& t) {
    const int k = v * C::NSL + c;
    hq = hk * p.G + hg * nh + k % nh;
    t = qb * nq + k / nh;
  };
  auto band_of = [&](int t, int& lo, int& hi) {
    lo = hi = 0;
    if (t < nqt) {
      lo = SPU * ds_kb_lo(t, p.window, nkb);
      hi = min(SPU * ds_kb_hi(t, p.causal, nkb), nsb);
      if (hi < lo) hi = lo;
    }
  };
  // the workgroup's band: the union over all slots (scalar)
  int g_lo = 0x7fffffff, g_hi = 0;
  for (int v = 0; v < C::NW; ++v)
    for (int c = 0; c < C::NSL; ++c) {
      int hq, t, lo, hi;
      slot_of(v, c, hq, t);
      band_of(t, lo, hi);
      if (hi > lo) {
        g_lo = min(g_lo, lo);
        g_hi = max(g_hi, hi);
      }
    }
  const int nsub = g_hi > g_lo ? g_hi - g_lo : 0;

  // This wave's slots.
  int hq_c[C::NSL], t_c[C::NSL], s_lo[C::NSL], s_hi[C::NSL];
  const char* dsrc[C::NSL];  // this lane's 16 bytes of the slot's first unit
  const T* kp = (const T*)a.k.data + b * a.k.sb + hk * a.k.sh;
#pragma unroll
  for (int c = 0; c < C::NSL; ++c) {
    slot_of(wave, c, hq_c[c], t_c[c]);
    band_of(t_c[c], s_lo[c], s_hi[c]);
    if (s_hi[c] > s_lo[c]) {
      const int64_t unit = (int64_t)(b * p.Hq + hq_c[c]) * a.ds_head +
                           ds_tile_offset(t_c[c], p.causal, p.window, nkb);
      dsrc[c] = a.ds + unit * kDsUnitB + lane * 16;
    } else {
      dsrc[c] = (const char*)kp;  // never used for data: a valid address to load from
    }
  }

  // Block-sparse maps: the block-map row of each of this wave's slots over
  // the workgroup's KV blocks, in (dynamic) LDS, so that the loop issues no
  // memory operation besides its own loads; in a walked sub-block, a slot
  // whose block is removed skips its MFMAs and loads a cached address
  // instead of its dS (the dK/dV kernel does not store removed units).
  extern __shared__ unsigned char sblk[];
  constexpr int SPB = kBlk / C::SB;  // sub-blocks per block
  const int kb0 = g_lo / SPB, nkbw = nsub > 0 ? (g_hi - 1) / SPB - kb0 + 1 : 0;
  unsigned char* myblk = sblk + wave * C::NSL * kBlkRowMax;
  if (p.blk) {
#pragma unroll
    for (int c = 0; c < C::NSL; ++c) {
      const unsigned char* row = block_row(p, b, hq_c[c], min(t_c[c] * kDsQT, p.Sq - 1));
      for (int i = lane; i < nkbw; i += 64) myblk[c * kBlkRowMax + i] = row[kb0 + i];
    }
  }
  auto live = [&](int c, int s) { return !p.blk || myblk[c * kBlkRowMax + s / SPB - kb0] != 0; };

  // Block-sparse maps (BLK): the sub-blocks some slot of the workgroup
  // computes (inside its band, block not removed), in order; the walk visits
  // only those (step i: sub-block g_lo + slist[i]).
  unsigned short* slist = (unsigned short*)(sblk + C::NW * C::NSL * kBlkRowMax);
  __shared__ int s_nlive;
  int nlive = nsub;
  if constexpr (BLK) {
    __syncthreads();  // every wave's block-map rows are in LDS
    if (wave == 0) {
      int base = 0;
      for (int i0 = 0; i0 < nsub; i0 += 64) {
        const int sb = g_lo + i0 + lane;
        bool any = false;
        if (i0 + lane < nsub) {
          for (int v = 0; v < C::NW && !any; ++v)
            for (int c = 0; c < C::NSL && !any; ++c) {
              int hq, t, lo, hi;
              slot_of(v, c, hq, t);
              band_of(t, lo, hi);
              any = sb >= lo && sb < hi && sblk[(v * C::NSL + c) * kBlkRowMax + sb / SPB - kb0] != 0;
            }
        }
        const unsigned long long m = __builtin_amdgcn_ballot_w64(any);
        if (any) slist[base + __builtin_popcountll(m & ((1ull << lane) - 1))] = (unsigned short)(i0 + lane);
        base += __builtin_popcountll(m);
      }
      if (lane == 0) s_nlive = base;
    }
    __syncthreads();
    nlive = __builtin_amdgcn_readfirstlane(s_nlive);
  }
  // sub-block of walk step i (i < nlive)
  auto sub_at = [&](int i) -> int {
    if constexpr (BLK) return g_lo + __builtin_amdgcn_readfirstlane((int)slist[i]);
    else return g_lo + i;
  };

  // K copies: chunk q = (wave EK + e) 64 + lane of the sub-block, row q / CPR,
  // at its swizzled chunk (the dual-use swizzle of the backward tiles).
  int krow[C::EK], kchk[C::EK];
#pragma unroll
  for (int e = 0; e < C::EK; ++e) {
    const int q = (wave * C::EK + e) * 64 + lane;
    krow[e] = q / C::CPR;
    kchk[e] = swz_dual_inv<C::CPR>(krow[e], q % C::CPR);
  }
  const unsigned lds0 = lds_addr_of(smem);
  auto issue_k = [&](int i) {  // K rows of walk step i (clamped to the last) into stage i % KSTAGES
    const int s = BLK ? sub_at(min(i, nlive - 1)) : min(g_lo + i, g_hi - 1);
    const unsigned sb = lds0 + (i & (C::KSTAGES - 1)) * C::KTILEB;
#pragma unroll
    for (int e = 0; e < C::EK; ++e) {
      const int64_t r = min(s * C::SB + krow[e], p.Skv - 1);
      load_lds16(kp + r * a.k.ss + kchk[e] * 8, sb + (wave * C::EK + e) * 1024);
    }
  };
  // dS of sub-block g_lo + i for the wave's slots into buf (NSL x KS operands)
  auto issue_ds = [&](int i, i32x4 (&buf)[C::NDS]) {
    const int s = i < nlive ? sub_at(i) : g_hi;  // past the end: outside every band (cached dummy loads)
#pragma unroll
    for (int c = 0; c < C::NSL; ++c) {
      const bool in = s >= s_lo[c] && s < s_hi[c] && live(c, s);
      const char* src = in ? dsrc[c] + (int64_t)(s / SPU - s_lo[c] / SPU) * kDsUnitB + (s % SPU) * C::SUBB
                           : dsrc[c];
#pragma unroll
      for (int f = 0; f < C::KS; ++f) load16_async(buf[c * C::KS + f], src + (in ? f * 1024 : 0));
    }
  };
  auto wait_ds = [&](i32x4 (&buf)[C::NDS], auto n_c) {
    constexpr int N = decltype(n_c)::value;
    static_assert(C::NDS == 4 || C::NDS == 8 || C::NDS == 16, "dS operand count");
    if constexpr (C::NDS == 4) {
      wait_vmcnt_tied<N>(buf[0], buf[1], buf[2], buf[3]);
    } else {
      wait_vmcnt_tied<N>(buf[0], buf[1], buf[2], buf[3], buf[4], buf[5], buf[6], buf[7]);
      if constexpr (C::NDS == 16)
        wait_vmcnt_tied<N>(buf[8], buf[9], buf[10], buf[11], buf[12], buf[13], buf[14], buf[15]);
    }
  };

  // Transpose-read offsets (A operands K^T: rows 4h + (lane % 16) / 4 and
  // + 8 of each 16-row k step, columns of d-block db).
  int voff_lo[C::DB], voff_hi[C::DB];
  {
    const int tr_row = 4 * h + ((lane & 15) >> 2);
    const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
    for (int db = 0; db < C::DB; ++db) {
      const int c = 4 * db + (tr_col >> 3), e2 = (tr_col & 7) * 2;
      voff_lo[db] = tr_row * C::ROWB + swz_dual<C::CPR>(tr_row, c) * 16 + e2;
      voff_hi[db] = (tr_row + 8) * C::ROWB + swz_dual<C::CPR>(tr_row + 8, c) * 16 + e2;
    }
  }

  f32x16 acc[C::NSL][C::DB];  // [slot][d-block]
#pragma unroll
  for (int c = 0; c < C::NSL; ++c)
#pragma unroll
    for (int db = 0; db < C::DB; ++db) acc[c][db] = f32x16{};

  i32x4 dsb[3][C::NDS];
#pragma unroll
  for (int j = 0; j < 3; ++j)
#pragma unroll
    for (int f = 0; f < C::NDS; ++f) dsb[j][f] = i32x4{0, 0, 0, 0};

  // Sub-block i: wait for its K rows and dS (the EK copies and NDS loads of
  // the newer issue step may stay in flight), then issue the copies of
  // i + KAHEAD and the loads of i + DAHEAD, then the MFMAs.
  auto step = [&](int i, auto bi_c) {
    constexpr int BI = decltype(bi_c)::value;
    constexpr int BN = (BI + C::DAHEAD) % 3;
    auto& cur = dsb[BI];
    wait_ds(cur, std::integral_constant<int, C::EK + C::NDS>{});
    __syncthreads();  // every wave's K copies of i landed; stage (i - 1) % 4 is free
    issue_k(i + C::KAHEAD);
    issue_ds(i + C::DAHEAD, dsb[BN]);
    const int s = sub_at(i);
    bool on[C::NSL];
#pragma unroll
    for (int c = 0; c < C::NSL; ++c) on[c] = s >= s_lo[c] && s < s_hi[c] && live(c, s);
    const char* sK = smem + (i & (C::KSTAGES - 1)) * C::KTILEB;
    // 16 (k step, d-block) operand reads, each feeding one MFMA per slot
    i16x4 alo[3], ahi[3];
    auto rdA = [&](int m, i16x4& lo, i16x4& hi) {  // k step m / DB, d-block m % DB
      const int off = 16 * (m / C::DB) * C::ROWB;
      lo = lds_read_tr4(sK + (voff_lo[m % C::DB] + off));
      hi = lds_read_tr4(sK + (voff_hi[m % C::DB] + off));
    };
    rdA(0, alo[0], ahi[0]);
    rdA(1, alo[1], ahi[1]);
#pragma unroll
    for (int m = 0; m < C::KS * C::DB; ++m) {
      __builtin_amdgcn_sched_barrier(0);
      if (m + 2 < C::KS * C::DB) rdA(m + 2, alo[(m + 2) % 3], ahi[(m + 2) % 3]);
      const V8 av = cat_tr<V8>(alo[m % 3], ahi[m % 3]);
      const int ks = m / C::DB, db = m % C::DB;
#pragma unroll
      for (int c = 0; c < C::NSL; ++c)
        if (on[c]) acc[c][db] = M::mma(av, as_v8<V8>(cur[c * C::KS + ks]), acc[c][db]);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  if (nlive > 0) {
    // prologue in the steady-state issue order: K 0, K 1, dS 0, K 2, dS 1
    issue_k(0);
    issue_k(1);
    issue_ds(0, dsb[0]);
    issue_k(2);
    issue_ds(1, dsb[1]);
    int i = 0;
    for (; i + 3 <= nlive; i += 3) {
      step(i, std::integral_constant<int, 0>{});
      step(i + 1, std::integral_constant<int, 1>{});
      step(i + 2, std::integral_constant<int, 2>{});
    }
    if (i < nlive) step(i, std::integral_constant<int, 0>{});
    if (i + 1 < nlive) step(i + 1, std::integral_constant<int, 1>{});
    // The copies and loads past the end land before anything else runs: the
    // loads' destination registers are named in the waits, so the compiler
    // keeps them allocated (a register reused while a load into it is in
    // flight would be overwritten when the load lands).
    wait_ds(dsb[0], std::integral_constant<int, 0>{});
    wait_ds(dsb[1], std::integral_constant<int, 0>{});
    wait_ds(dsb[2], std::integral_constant<int, 0>{});
  }

  const float sc = p.scale;
#pragma unroll
  for (int c = 0; c < C::NSL; ++c) {
    const int my_m = t_c[c] * kDsQT + l32;
    if (t_c[c] < nqt && my_m < p.Sq) {
      T* out = (T*)a.dq.data + b * a.dq.sb + hq_c[c] * a.dq.sh + (int64_t)my_m * a.dq.ss + 4 * h;
#pragma unroll
      for (int db = 0; db < C::DB; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          st_global8(out + 32 * db + 8 * i, pack4<T>(acc[c][db][4 * i] * sc, acc[c][db][4 * i + 1] * sc,
                                                   acc[c][db][4 * i + 2] * sc, acc[c][db][4 * i + 3] * sc));
    }
  }
}

template <class T, int D>
hipError_t launch_dq_ds(const BwdArgs& a, hipStream_t st) {
  using C = DqsCfg<D>;
  BwdArgs x = a;
  const int nh = (a.p.G % 4 == 0) ? 4 : (a.p.G % 2 == 0) ? 2 : 1;
  const int nq = C::SLOTS / nh;
  const int nqt = (a.p.Sq + kDsQT - 1) / kDsQT;
  const int nqb = (nqt + nq - 1) / nq;
  x.ntiles = (nqb << 8) | nh;
  const dim3 grid(nqb * (a.p.G / nh) * a.p.B * a.p.Hkv), block(C::NW * 64);
  // block-sparse maps: block-map rows of the slots, then the sub-block walk list
  const int nsb = (a.p.Skv + C::SB - 1) / C::SB;
  if (a.p.blk) {
    const size_t dyn = (size_t)C::NW * C::NSL * kBlkRowMax + 2 * (size_t)(nsb + 2);
    hipLaunchKernelGGL((bwd_dq_ds_kernel<T, D, true>), grid, block, dyn, st, x);
  } else {
    hipLaunchKernelGGL((bwd_dq_ds_kernel<T, D, false>), grid, block, 0, st, x);
  }
  return hipGetLastError();
}

#define FLEXATT_DQ_DS_LAUNCHERS(D)                                                                     \
  hipError_t bwd_dq_ds_bf16_d##D(const BwdArgs& a, hipStream_t st) { return launch_dq_ds<__bf16, D>(a, st); } \
  hipError_t bwd_dq_ds_f16_d##D(const BwdArgs& a, hipStream_t st) { return launch_dq_ds<_Float16, D>(a, st); }
#if FLEXATT_D == 128
FLEXATT_DQ_DS_LAUNCHERS(128)
#elif FLEXATT_D == 64
FLEXATT_DQ_DS_LAUNCHERS(64)
#else
FLEXATT_DQ_DS_LAUNCHERS(256)
#endif

#endif  // FLEXATT_D == 128 || FLEXATT_D == 64 || FLEXATT_D == 256

}  // namespace flexatt
