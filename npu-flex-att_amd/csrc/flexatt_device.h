// Device-side building blocks shared by the flash-attention kernels (gfx950).
//
// Conventions used by every kernel in this library
//  * tensors are [B, H, S, D] with element strides; the innermost stride is 1
//    and rows start on 16-byte boundaries (the host entry points check this);
//  * scores are kept in the log2 domain: y = x * log2(e), so softmax weights
//    are exp2(y - m) and LSE(natural) = (m + log2(l)) * ln(2);
//  * MFMA 32x32x16 (bf16/fp16) lane layout, verified on MI355X:
//      A operand  lane l holds A[row = l%32][k = 8*(l/32) + t], t = 0..7
//      B operand  lane l holds B[k = 8*(l/32) + t][col = l%32]
//      C/D        acc[4*i + j] = C[row = 8*i + 4*(l/32) + j][col = l%32]
//  * ds_read_b64_tr_b16, per 16-lane group: with M[r][c] the c-th 16-bit
//    element at lane r's address, lane i receives M[4*t + i/4][i%4], t=0..3.
//    Pointing lane r at &X[k0 + r/4][n0 + 4*(r%4)] therefore hands lane i the
//    column X[k0 .. k0+3][n0 + i]: a transposed operand read from a row-major
//    LDS tile.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/flexatt.h"

namespace flexatt {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kPosInf = __builtin_huge_valf();

// Kernel-side view of one [B, H, S, D] tensor.
struct View {
  const void* data;
  int64_t sb, sh, ss;  // element strides (innermost stride is 1)
};
struct MutView {
  void* data;
  int64_t sb, sh, ss;
};

// Problem scalars shared by all kernels.
struct Shape {
  int B, Hq, Hkv, G, Sq, Skv;
  float scale;        // softmax scale
  float scale_log2;   // scale * log2(e)
  int causal;
  int window;         // 0 = off
  float cap;          // 0 = off
  float inv_cap;
  float tanh_k;       // 2 log2(e) scale / cap: exp2(s * tanh_k) = e^(2 scale s / cap)
  float cap_log2;     // cap * log2(e)
  const float* alibi;  // [Hq] or nullptr
  const int* doc;      // row bounds [B][Sq][2]: keys [lo, hi) query row i may attend, or nullptr
  const int* docc;     // column bounds [B][Skv][2]: query rows [lo, hi) that may attend key j
                       // (the same array as doc for a symmetric mask), or nullptr
  const unsigned char* blk;  // block map [B][blk_h][blk_nq][blk_nk] of 128 x 128 blocks, or nullptr
  int blk_h, blk_nq, blk_nk;
};

// --- element traits ----------------------------------------------------------
template <class T> struct Mfma;
template <> struct Mfma<__bf16> {
  typedef bf16x8 v8;
  static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma<_Float16> {
  typedef f16x8 v8;
  static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template <class T> __device__ __forceinline__ T from_f32(float x) { return (T)x; }
template <class T> __device__ __forceinline__ float to_f32(T x) { return (float)x; }

// --- small helpers -------------------------------------------------------------
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// acc *= s in place.  Written with tied asm operands so that a rescale under a
// branch leaves the accumulator in its registers (a plain multiply makes the
// register allocator copy the whole accumulator on the other path).
__device__ __forceinline__ void scale_inplace(f32x16& a, float s) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    float x = a[r];
    asm volatile("v_mul_f32_e32 %0, %1, %0" : "+v"(x) : "v"(s));
    a[r] = x;
  }
}

// Register fence: the value must be computed before this point and is read
// again after it.  Volatile asm keeps its place relative to barriers, so this
// stops the compiler from sinking a phase's results past a workgroup barrier
// (or hoisting their consumers before it).
template <class X>
__device__ __forceinline__ void pin(X& x) {
  asm volatile("" : "+v"(x));
}
// Read-only form: x must be in a VGPR at this point (e.g. read out of an
// accumulator register here), without a copy for the later uses.
template <class X>
__device__ __forceinline__ void pin_in(const X& x) {
  asm volatile("" ::"v"(x));
}

// --- direct global -> LDS tile staging --------------------------------------
// global_load_lds_dwordx4: lane l's 16 bytes land at LDS byte address
// (lds_addr + 16 * l).  Issued through asm so that the compiler does not place
// a full vmcnt(0) wait before every later LDS access; completion is tracked
// by the caller with wait_vmcnt<N>() followed by a workgroup barrier (vector
// memory operations retire in order, so the compiler's own waits stay valid,
// only more conservative).
__device__ __forceinline__ void load_lds16(const void* gptr, unsigned lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(lds_addr) : "memory");
}
// Same for one dword per lane (lane l's 4 bytes land at lds_addr + 4 * l).
__device__ __forceinline__ void load_lds4(const void* gptr, unsigned lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(gptr), "s"(lds_addr) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// 16 bytes global -> registers, issued through asm like load_lds16 so that
// the compiler's wait counting does not see it; the data may be read only
// after wait_vmcnt_tied<N>(...) names the destination registers (the tie
// keeps every use of them after the wait).  The compiler does not know the
// load is in flight, so a kernel that uses it must keep the destination
// registers in place: one that spills VGPRs may store such a register to
// scratch and reuse it before the load lands (the landing load then
// overwrites whatever the register holds by then).  build_lib.py rejects a
// build in which a kernel of such a source uses scratch.
__device__ __forceinline__ void load16_async(i32x4& dst, const void* gptr) {
  asm volatile("global_load_dwordx4 %0, %1, off" : "+v"(dst) : "v"(gptr) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt_tied(i32x4& a, i32x4& b, i32x4& c, i32x4& d, i32x4& e, i32x4& f,
                                                i32x4& g, i32x4& h) {
  asm volatile("s_waitcnt vmcnt(%8)"
               : "+v"(a), "+v"(b), "+v"(c), "+v"(d), "+v"(e), "+v"(f), "+v"(g), "+v"(h)
               : "n"(N)
               : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt_tied(i32x4& a, i32x4& b, i32x4& c, i32x4& d) {
  asm volatile("s_waitcnt vmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "n"(N) : "memory");
}
__device__ __forceinline__ unsigned lds_addr_of(const void* p) {
  return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// Swizzled, unpadded tile layouts (rows of CPR 16-byte chunks).  K tiles are
// read with 16-byte column reads (A rows of S^T = K Q^T); V/K^T/Q^T/dO^T
// tiles with the transpose read.  Both map logical chunk c of row r to a
// physical chunk within the same row, so whole tiles can be copied with
// 1 KB direct-to-LDS loads.  The maps were chosen by measured LDS throughput.
template <int CPR>
__device__ __forceinline__ int swz_col(int r, int c) {  // for 16-byte column reads
  if constexpr (CPR == 4) return c ^ ((r >> 2) & 3);
  else if constexpr (CPR == 8) return c ^ ((r >> 1) & 7);
  else return c ^ (r & 15);
}
template <int CPR>
__device__ __forceinline__ int swz_tr(int r, int c) {  // for transpose reads
  if constexpr (CPR == 4) return c;
  else if constexpr (CPR == 8) return (c + 4 * ((r >> 1) & 1)) & 7;
  else return (c + 4 * r) & (CPR - 1);
}
template <int CPR>
__device__ __forceinline__ int swz_tr_inv(int r, int p) {
  if constexpr (CPR == 4) return p;
  else if constexpr (CPR == 8) return (p - 4 * ((r >> 1) & 1)) & 7;
  else return (p - 4 * r) & (CPR - 1);
}

// One layout for tiles that are read both ways: 16-byte row reads (rows as
// MFMA operands; 16 lanes per LDS cycle read one chunk of 16 consecutive
// rows) and transpose reads (32 lanes per LDS cycle read chunks 4j..4j+3 of
// 4 consecutive rows 4i..4i+3).  The LDS serves 64 banks x 4 bytes, i.e. 16
// groups of 16 bytes, per cycle.  Chunk c of row r sits at chunk c ^ g(r):
//  * 256-byte rows (CPR 16, one row per bank row): g(r) = (r mod 4) * 4 +
//    (r / 4) mod 4 is a permutation over any 16 consecutive rows (row reads
//    hit 16 distinct groups) and 4 consecutive rows differ in the top two
//    bits of g (a transpose read's 16 chunks land in 16 distinct groups);
//  * 128-byte rows (CPR 8, rows 2i and 2i+1 share a bank row, group
//    8 (r mod 2) + chunk): g(r) = 4 r1 + 2 r3 + r2 (r = r3 r2 r1 r0 in
//    binary) is a permutation over the 8 rows of one parity in any aligned
//    16 rows, and rows 4i, 4i+2 (and 4i+1, 4i+3) differ in bit 2 of g, so
//    their 4-chunk groups fall in different halves of the bank row.
// The swizzle is its own inverse.
//  * 512-byte rows (CPR 32, a row spans two bank rows, group = chunk mod
//    16): the CPR 16 map on the low four chunk bits.
template <int CPR>
__device__ __forceinline__ int swz_dual(int r, int c) {
  static_assert(CPR == 32 || CPR == 16 || CPR == 8, "dual-use swizzle is defined for 512-, 256- and 128-byte rows");
  if constexpr (CPR >= 16) return c ^ (((r & 3) << 2) | ((r >> 2) & 3));
  else return c ^ ((((r >> 1) & 1) << 2) | (((r >> 3) & 1) << 1) | ((r >> 2) & 1));
}
template <int CPR>
__device__ __forceinline__ int swz_dual_inv(int r, int p) {
  return swz_dual<CPR>(r, p);
}

// Value of lane l ^ 32 (the other half of the wave).
__device__ __forceinline__ float swap_halves(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const bool lo = (threadIdx.x & 32) == 0;
  return __uint_as_float(lo ? r[1] : r[0]);
}

__device__ __forceinline__ i32x4 ld_global16(const void* p) { return *(const i32x4*)p; }
__device__ __forceinline__ void st_global8(void* p, i32x2 v) { *(i32x2*)p = v; }

__device__ __forceinline__ i32x4 lds_read16(const void* p) {
  return *(const __attribute__((address_space(3))) i32x4*)((__attribute__((address_space(3))) char*)p);
}

// Transposed 4 x 16-bit read (see header comment).
__device__ __forceinline__ i16x4 lds_read_tr4(const void* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4*)((__attribute__((address_space(3))) char*)p));
}

template <class V8> __device__ __forceinline__ V8 as_v8(i32x4 x) { return __builtin_bit_cast(V8, x); }
template <class V8> __device__ __forceinline__ V8 cat_tr(i16x4 a, i16x4 b) {
  i16x8 r = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  return __builtin_bit_cast(V8, r);
}

// Pack 8 fp32 accumulator values (acc[o..o+7]) into an MFMA operand.
template <class T>
__device__ __forceinline__ typename Mfma<T>::v8 pack8(const f32x16& a, int o) {
  typename Mfma<T>::v8 r;
#pragma unroll
  for (int t = 0; t < 8; ++t) r[t] = from_f32<T>(a[o + t]);
  return r;
}

// max of two / three floats as single instructions.  fmaxf would first
// quiet each operand (one extra instruction per input in IEEE mode); these
// are only used where the inputs are scores, for which the NaN behaviour of
// the plain instruction (a quiet NaN input is ignored) is acceptable.
__device__ __forceinline__ float max2(float a, float b) {
  float r;
  asm("v_max_f32_e32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float max3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
// Max of 16 accumulator values as 7 instructions, leaving two partials.
__device__ __forceinline__ void max16_partial(const f32x16& s, float& f, float& g) {
  const float a = max3(s[0], s[1], s[2]), b = max3(s[3], s[4], s[5]), c = max3(s[6], s[7], s[8]);
  const float d = max3(s[9], s[10], s[11]), e = max3(s[12], s[13], s[14]);
  f = max3(a, b, c);
  g = max3(d, e, s[15]);
}

// acc + sum of the 8 16-bit values of an MFMA operand (fp32 accumulate).
template <class T> struct Dot2;
template <> struct Dot2<__bf16> {
  typedef __bf16 x2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ float add(x2 a, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(a, x2{(__bf16)1.0f, (__bf16)1.0f}, c, false);
  }
};
template <> struct Dot2<_Float16> {
  typedef _Float16 x2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ float add(x2 a, float c) {
    return __builtin_amdgcn_fdot2(a, x2{(_Float16)1.0f, (_Float16)1.0f}, c, false);
  }
};
template <class T>
__device__ __forceinline__ void sum8(typename Mfma<T>::v8 p, float (&acc)[4]) {
  acc[0] = Dot2<T>::add(__builtin_shufflevector(p, p, 0, 1), acc[0]);
  acc[1] = Dot2<T>::add(__builtin_shufflevector(p, p, 2, 3), acc[1]);
  acc[2] = Dot2<T>::add(__builtin_shufflevector(p, p, 4, 5), acc[2]);
  acc[3] = Dot2<T>::add(__builtin_shufflevector(p, p, 6, 7), acc[3]);
}

// Two fp32 values rounded to T, packed into one 32-bit word (a in the low half).
template <class T>
__device__ __forceinline__ unsigned pk2(float a, float b) {
  typedef T x2 __attribute__((ext_vector_type(2)));
  const x2 v = {from_f32<T>(a), from_f32<T>(b)};
  return __builtin_bit_cast(unsigned, v);
}

// Pack 4 fp32 values into 4 x T (8 bytes) for a store.
template <class T>
__device__ __forceinline__ i32x2 pack4(float a, float b, float c, float d) {
  T v[4] = {from_f32<T>(a), from_f32<T>(b), from_f32<T>(c), from_f32<T>(d)};
  return __builtin_bit_cast(i32x2, v);
}

// Remap the linear workgroup id so that each XCD (dispatch is round-robin over
// the 8 XCDs) receives a contiguous range of logical work items: items that
// share K/V then share one L2.
__device__ __forceinline__ int xcd_remap(int w, int n) {
  if ((n & 7) != 0) return w;
  return (w & 7) * (n >> 3) + (w >> 3);
}

// Work-item order for gfx950's workgroup dispatch: workgroup i runs on XCD
// i % 8, and within an XCD consecutive workgroups go to its four shader
// engines in a fixed rotation; a workgroup waits for a free CU on its own
// engine and holds back every later one.  The grid is ng groups (items that
// share K/V) x nk items per group, item k = 0 the longest.  Each XCD takes
// ng / 8 whole groups (one L2), deals their items longest first across the
// groups, and reverses every other run of four, so that the four engines get
// the same mix of lengths and free their CUs together (longest first within
// each engine).  False when ng is not a multiple of 8 (caller's own order).
// Slot (work-item ordinal) of this workgroup: its own index, or, past the
// first nstatic workgroups (one per CU) when a queue counter is given, the
// next unclaimed slot, so that workgroups starting early (on faster XCDs)
// take the longest remaining items.  Every thread of the workgroup calls it.
__device__ __forceinline__ int queue_slot(int* queue, int nstatic) {
  if (!queue || (int)blockIdx.x < nstatic) return blockIdx.x;
  __shared__ int slot;
  if (threadIdx.x == 0) slot = nstatic + atomicAdd(queue, 1);
  __syncthreads();
  return __builtin_amdgcn_readfirstlane(slot);
}

__device__ __forceinline__ bool xcd_lpt_item(int i, int nk, int ng, int& k, int& g) {
  if ((ng & 7) != 0) return false;
  const int x = i & 7, j = i >> 3;
  const int gx = ng >> 3, nx = gx * nk;
  const int m = j >> 2, r = j & 3;
  const int s = ((m & 1) && 4 * m + 3 < nx) ? 4 * m + 3 - r : j;
  k = s / gx;
  g = x * gx + s % gx;
  return true;
}

// Score transform in the log2 domain for one element: scale, soft-cap, ALiBi
// (dij = i - j as a float; exact for |i - j| < 2^24).
template <bool SOFTCAP, bool ALIBI>
__device__ __forceinline__ float score_log2_d(float s, const Shape& p, float slope_log2, float dij, float& t) {
  float y;
  if constexpr (SOFTCAP) {
    // tanh(x) = 1 - 2 / (e^(2x) + 1) with x = scale s / cap; y = cap log2(e) tanh(x)
    // straight from the reciprocal (t is only formed where the caller reads it)
    const float r = fast_rcp(fast_exp2(s * p.tanh_k) + 1.0f);
    t = __builtin_fmaf(-2.0f, r, 1.0f);
    y = __builtin_fmaf(-2.0f * p.cap_log2, r, p.cap_log2);
  } else {
    y = s * p.scale_log2;
  }
  if constexpr (ALIBI) y = __builtin_fmaf(slope_log2, dij, y);
  return y;
}
template <bool SOFTCAP, bool ALIBI>
__device__ __forceinline__ float score_log2(float s, const Shape& p, float slope_log2, int i, int j, float& t) {
  return score_log2_d<SOFTCAP, ALIBI>(s, p, slope_log2, (float)(i - j), t);
}

// Interval masks (document masks, PrefixLM): the keys [lo, hi) query row i
// of batch b may attend; [0, INT_MAX) when off.  Both bounds are
// non-decreasing in i, so those of a range's first and last rows bound the
// whole range.
__device__ __forceinline__ void doc_bounds(const Shape& p, int b, int i, int& lo, int& hi) {
  if (p.doc) {
    const int* d = p.doc + ((int64_t)b * p.Sq + i) * 2;
    lo = d[0];
    hi = d[1];
  } else {
    lo = 0;
    hi = 0x7fffffff;
  }
}
// The transpose: the query rows [lo, hi) that may attend key j (for the
// KV-stationary kernels); non-decreasing in j as well.
__device__ __forceinline__ void col_bounds(const Shape& p, int b, int j, int& lo, int& hi) {
  if (p.docc) {
    const int* d = p.docc + ((int64_t)b * p.Skv + j) * 2;
    lo = d[0];
    hi = d[1];
  } else {
    lo = 0;
    hi = 0x7fffffff;
  }
}
// Block-sparse mask: whether the 128 x 128 block holding (query row i, key j)
// of head hq is computed (true when no block map is set).
constexpr int kBlk = 128;
constexpr int kBlkRowMax = 2048;  // KV blocks a kernel keeps of one block-map row (Skv <= 256 Ki)
__device__ __forceinline__ const unsigned char* block_row(const Shape& p, int b, int hq, int i) {
  return p.blk + ((int64_t)(b * p.blk_h + (p.blk_h > 1 ? hq : 0)) * p.blk_nq + i / kBlk) * p.blk_nk;
}
__device__ __forceinline__ bool block_on(const Shape& p, int b, int hq, int i, int j) {
  return !p.blk || block_row(p, b, hq, i)[j / kBlk] != 0;
}

// --- staged dS (the D = 128 backward) -----------------------------------------
// The dK/dV kernel writes the dS it feeds its own MFMAs (rounded to the input
// dtype, without the softmax scale) to a workspace, and the dQ kernel forms
// dQ = scale * dS K from it without recomputing S and dP.  The unit is one
// (query tile of 32 rows, KV block of 128 rows) pair of one query head:
// 8 fragments of 1 KB, fragment f holding KV rows 16 f .. 16 f + 15 as the
// B operand of a 32x32x16 MFMA: lane l, element e is query row l % 32 and KV
// row 16 f + 4 (l / 32) + e (e < 4), 16 f + 8 + 4 (l / 32) + e - 4 (e >= 4)
// (the k order of the K^T transpose reads).  Only the pairs inside the
// causal / window band are stored: query tile t holds KV blocks
// [ds_kb_lo(t), ds_kb_hi(t)), the tiles of one head follow each other in t
// order, and the heads in (b, h) order.
constexpr int kDsQT = 32;     // query rows per dS unit
constexpr int kDsKB = 128;    // KV rows per dS unit
constexpr int kDsUnitB = 8192;  // bytes per dS unit (16-bit elements)
// fp32 inputs stage dS in fp32 over the same units (32 query rows x 128 KV
// rows, same band and offsets), laid out as 4 slices of 32 KV rows, each
// [query row][KV row] row-major: element (i, j) of the unit at
// ((j / 32) * 32 + i) * 32 + j % 32.
constexpr int kDsUnitB32 = 16384;

__host__ __device__ __forceinline__ int ds_kb_lo(int t, int window, int nkb) {
  if (window <= 0) return 0;
  const int x = kDsQT * t - window;  // first key row any row of the tile keeps
  const int lo = x > 0 ? x / kDsKB : 0;
  return lo < nkb ? lo : nkb;
}
__host__ __device__ __forceinline__ int ds_kb_hi(int t, int causal, int nkb) {
  if (!causal) return nkb;
  const int hi = t / (kDsKB / kDsQT) + 1;  // last key row of the tile is 32 t + 31
  return hi < nkb ? hi : nkb;
}
// sum over u in [0, x) of min(n, floor(u / 4)) (0 for x <= 0)
__host__ __device__ __forceinline__ int64_t ds_quarter_sum(int64_t x, int64_t n) {
  if (x <= 0) return 0;
  if (x <= 4 * n) {
    const int64_t q = x >> 2, r = x & 3;
    return 2 * q * (q - 1) + r * q;
  }
  return 2 * n * (n - 1) + (x - 4 * n) * n;
}
// Units stored for query tiles [0, t) of one head: the sum of
// ds_kb_hi - ds_kb_lo, in closed form (kb_hi = min(nkb, t/4 + 1) and
// kb_lo = min(nkb, max(0, floor((t - ceil(W/32)) / 4))) are clamped quarter
// steps).
__host__ __device__ __forceinline__ int64_t ds_tile_offset(int t, int causal, int window, int nkb) {
  static_assert(kDsKB == 4 * kDsQT, "closed form assumes four query tiles per KV block");
  const int64_t hi = causal ? ds_quarter_sum((int64_t)t + 4, nkb) : (int64_t)t * nkb;
  const int64_t lo = window > 0 ? ds_quarter_sum((int64_t)t - (window + kDsQT - 1) / kDsQT, nkb) : 0;
  return hi - lo;
}

// allowed(i, j) for the masks of the path (j < Skv is the KV tail).
__device__ __forceinline__ bool allowed(const Shape& p, int i, int j) {
  bool ok = j < p.Skv;
  if (p.causal) ok = ok && (j <= i);
  if (p.window > 0) ok = ok && (i - j <= p.window);
  return ok;
}

}  // namespace flexatt
