// Fused 4-bit dequant-GEMV for gfx950 (MI355X), batch 1..16, and the device decoder.
//
// Work unit = one (16-row tile, 512-element span) block of the device stream
// (fourbit_layout.h).  Lane L of a wave loads the 96-byte (GF4) / 68-byte (E2M1) record
// of row 16t + L%16, item 4sp + L/16, decodes it in registers -- GF4: two v_perm_b32
// lookups per byte plane merged by XOR; E2M1: v_cvt_scalef32_pk_{bf16,f16}_fp4 -- into
// exactly the A operand of v_mfma_f32_16x16x32_{f16,bf16}, and the matrix core does the
// multiply-accumulate against x (B operand, one batch row per MFMA column, staged in
// LDS).  The VALU only decodes; the cross-lane reduction is the MFMA itself; batch 1..16
// costs the same VALU work.
//
// Partition: workgroup g (16 waves, one per CU; for small batch-1 layers 8 waves, two per
// CU) owns the contiguous 16-row tiles [t0, t1).
// Its (tile, span) units are handed to its waves through an LDS counter: the SIMDs issue
// the oldest wave first, so with a fixed split the youngest wave of each SIMD would finish
// long after the others; taking units on demand keeps all waves busy to the end.  Each
// unit's partial sums go to a slot of their own, and the wave that finishes a row tile's
// last unit adds each of its outputs' slots in span order, so results do not depend on
// which wave did what.
// When x does not fit LDS the K range is cut into S slices staged one after the other, or
// (kSpanX, batches of 2-16) each wave stages the x of its own spans, one at a time.
// No workgroup talks to another: no global atomics or device-scope fences.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <atomic>
#include <type_traits>

#include "fourbit.h"
#include "fourbit_layout.h"

// The library's GEMV is two translation units.  fourbit_gemv_ilp.hip includes this file with
// FB_GEMV_ILP_TU defined and is compiled with the compiler's max-ILP instruction scheduling;
// it holds the kernels that run faster that way, the 8-wave batch-1 ones (kFlat1 and the
// rotated kRot1, one workgroup per CU), and fb_ilp::launch starts them.  Every
// other kernel stays here: with max-ILP scheduling the 16-wave batch-1 kernel ran the large
// layers 1.4-1.8 us slower.
namespace fb_ilp {
// A plan's fields are passed one by one: the plan type is local to each unit.  Not part of
// the library's ABI.
__attribute__((visibility("hidden"))) int launch(int fmt, int xdt, int mode, const void* wdev, const void* x, void* y,
           const fb_shape_t* s, int grid, int SPL, int GS, int tq, int tr, int S, size_t lds,
           int xp, hipStream_t stream);
}  // namespace fb_ilp

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf168_t __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 16;  // waves of a full-CU workgroup
constexpr int kLdsLimit = 160 * 1024;
constexpr int kSliceBytes = 272;  // 128 x 16-bit values + 16-byte pad (bank spread)

// ---------------------------------------------------------------------------------
// small device helpers
// ---------------------------------------------------------------------------------
__device__ __forceinline__ unsigned perm(unsigned s0, unsigned s1, unsigned sel) {
  return __builtin_amdgcn_perm(s0, s1, sel);
}

__device__ __forceinline__ u32x4 ldg16(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

__device__ __forceinline__ void store_y(void* y, int64_t idx, float v, int ydt) {
  if (ydt == FB_DT_F32) {
    static_cast<float*>(y)[idx] = v;
  } else if (ydt == FB_DT_F16) {
    static_cast<_Float16*>(y)[idx] = (_Float16)v;
  } else {
    static_cast<__bf16*>(y)[idx] = (__bf16)v;
  }
}

// n / d for 0 <= n < 2^30 and 1 <= d < 2^16, with m = div_magic(d) from the host: the high
// half of n * m is n / d or one less, and one compare fixes it.  Used instead of integer
// division, which is a long instruction sequence on this GPU.
__device__ __forceinline__ int fdiv(int n, int d, unsigned m) {
  const int q = (int)__umulhi((unsigned)n, m);
  return (q + 1) * d <= n ? q + 1 : q;
}

// n / d for 0 <= n < 2^20 and 1 <= d < 2^20 through the fp32 reciprocal: the truncated
// product is within one of the quotient, and two compares fix it.  Prologue code uses it
// instead of integer division, which is a long scalar sequence that every wave of a
// workgroup would run on the CU's one scalar unit.
__device__ __forceinline__ int small_div(int n, int d) {
  int q = (int)((float)n * __builtin_amdgcn_rcpf((float)d));
  q -= q * d > n ? 1 : 0;
  q += (q + 1) * d <= n ? 1 : 0;
  return q;
}

// GF4 decode of one 32-bit word (8 codes, layout order) into 4 fp16 pairs in element
// order (e0,e1) (e2,e3) (e4,e5) (e6,e7).  tl/th: lo/hi byte-plane tables
// {A'[0..3], A'[4..7], B'[0..3], B'[4..7]}.
__device__ __forceinline__ u32x4 gf4_decode8(unsigned q, const u32x4& tl, const u32x4& th) {
  const unsigned sa = q & 0x0F0F0F0Fu;
  const unsigned sb = (q >> 4) & 0x0F0F0F0Fu;
  const unsigned sa8 = sa ^ 0x08080808u;
  const unsigned sb8 = sb ^ 0x08080808u;
  const unsigned loA = perm(tl.y, tl.x, sa) ^ perm(tl.w, tl.z, sa8);
  const unsigned hiA = perm(th.y, th.x, sa) ^ perm(th.w, th.z, sa8);
  const unsigned loB = perm(tl.y, tl.x, sb) ^ perm(tl.w, tl.z, sb8);
  const unsigned hiB = perm(th.y, th.x, sb) ^ perm(th.w, th.z, sb8);
  u32x4 w;
  w.x = perm(hiA, loA, 0x05010400u);
  w.y = perm(hiA, loA, 0x07030602u);
  w.z = perm(hiB, loB, 0x05010400u);
  w.w = perm(hiB, loB, 0x07030602u);
  return w;
}

// Two independent 8-code decodes written stage by stage, so the scheduler sees twice the
// instruction-level parallelism of one decode chain.
__device__ __forceinline__ void gf4_decode16(unsigned q0, unsigned q1, const u32x4& tl,
                                             const u32x4& th, u32x4& w0, u32x4& w1) {
  const unsigned sa0 = q0 & 0x0F0F0F0Fu, sa1 = q1 & 0x0F0F0F0Fu;
  const unsigned t0 = q0 >> 4, t1 = q1 >> 4;
  const unsigned sa80 = sa0 ^ 0x08080808u, sa81 = sa1 ^ 0x08080808u;
  const unsigned sb0 = t0 & 0x0F0F0F0Fu, sb1 = t1 & 0x0F0F0F0Fu;
  const unsigned sb80 = sb0 ^ 0x08080808u, sb81 = sb1 ^ 0x08080808u;
  const unsigned la0 = perm(tl.y, tl.x, sa0), la1 = perm(tl.y, tl.x, sa1);
  const unsigned lb0 = perm(tl.w, tl.z, sa80), lb1 = perm(tl.w, tl.z, sa81);
  const unsigned ha0 = perm(th.y, th.x, sa0), ha1 = perm(th.y, th.x, sa1);
  const unsigned hb0 = perm(th.w, th.z, sa80), hb1 = perm(th.w, th.z, sa81);
  const unsigned loA0 = la0 ^ lb0, loA1 = la1 ^ lb1, hiA0 = ha0 ^ hb0, hiA1 = ha1 ^ hb1;
  const unsigned lc0 = perm(tl.y, tl.x, sb0), lc1 = perm(tl.y, tl.x, sb1);
  const unsigned ld0 = perm(tl.w, tl.z, sb80), ld1 = perm(tl.w, tl.z, sb81);
  const unsigned hc0 = perm(th.y, th.x, sb0), hc1 = perm(th.y, th.x, sb1);
  const unsigned hd0 = perm(th.w, th.z, sb80), hd1 = perm(th.w, th.z, sb81);
  w0.x = perm(hiA0, loA0, 0x05010400u); w1.x = perm(hiA1, loA1, 0x05010400u);
  w0.y = perm(hiA0, loA0, 0x07030602u); w1.y = perm(hiA1, loA1, 0x07030602u);
  const unsigned loB0 = lc0 ^ ld0, loB1 = lc1 ^ ld1, hiB0 = hc0 ^ hd0, hiB1 = hc1 ^ hd1;
  w0.z = perm(hiB0, loB0, 0x05010400u); w1.z = perm(hiB1, loB1, 0x05010400u);
  w0.w = perm(hiB0, loB0, 0x07030602u); w1.w = perm(hiB1, loB1, 0x07030602u);
}

// E2M1 decode of one 32-bit word (8 codes, canonical order) times `scale`.
template <int XDT>
__device__ __forceinline__ u32x4 e2m1_decode8(unsigned q, float scale) {
  u32x4 w;
  if constexpr (XDT == FB_DT_BF16) {
    w.x = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, scale, 0));
    w.y = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, scale, 1));
    w.z = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, scale, 2));
    w.w = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, scale, 3));
  } else {
    w.x = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q, scale, 0));
    w.y = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q, scale, 1));
    w.z = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q, scale, 2));
    w.w = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q, scale, 3));
  }
  return w;
}

template <int XDT>
__device__ __forceinline__ f32x4 mfma(const u32x4& a, const u32x4& b, const f32x4& c) {
  if constexpr (XDT == FB_DT_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf168_t, a),
                                                   __builtin_bit_cast(bf168_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a),
                                                  __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
  }
}

// One lane's record of a work unit.
template <int FMT>
struct Rec {
  u32x4 nib[4];
  u32x4 t0, t1;  // GF4: lo / hi tables.  E2M1: t0.x holds the 4 scale bytes.
};

typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;  // raw (untyped) buffer, gfx9 family
constexpr int kNT = 2;                  // streaming (non-temporal) cache policy
// a buffer offset past every resource's range: the load returns zeros and moves no data
constexpr unsigned kXOutOfRange = 0x7FFFFFF0u;

// Loads one lane's record of the block at byte offset `boff` of the weight stream.
// With a zero-sized resource the loads are out of range: they return zeros and move no
// data, which is how the pipeline issues its loads unconditionally past the last unit.
// The tables / scales are issued first: chunk 0 can then be decoded as soon as they and
// nibble chunk 0 have arrived, while chunks 1..3 are still in flight.
template <int FMT>
__device__ __forceinline__ void load_rec(rsrc_t rs, unsigned boff, int lane, Rec<FMT>& r) {
  const int vo = lane * 16;
  if constexpr (FMT == FB_FMT_GF4) {
    r.t0 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, vo, (int)boff + 4096, kNT));
    r.t1 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, vo, (int)boff + 5120, kNT));
  } else {
    r.t0.x = __builtin_amdgcn_raw_buffer_load_b32(rs, lane * 4, (int)boff + 4096, kNT);
  }
#pragma unroll
  for (int c = 0; c < 4; ++c)
    r.nib[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             rs, vo + c * 1024, (int)boff, kNT));
}

// Record read for the device decoder (plain global loads).
template <int FMT>
__device__ __forceinline__ void load_rec_global(const uint8_t* __restrict__ blk, int lane,
                                                Rec<FMT>& r) {
  const uint8_t* base = blk + lane * 16;
#pragma unroll
  for (int c = 0; c < 4; ++c) r.nib[c] = ldg16(base + c * 1024);
  if constexpr (FMT == FB_FMT_GF4) {
    r.t0 = ldg16(base + 4096);
    r.t1 = ldg16(base + 5120);
  } else {
    r.t0.x = __builtin_nontemporal_load(reinterpret_cast<const unsigned*>(blk + 4096 + lane * 4));
  }
}

// ---------------------------------------------------------------------------------
// Activation staging.  The slice [k0, k0 + 512*SPL) of each batch row b is stored as
// 128-value groups of kSliceBytes: byte offset b*RS + (k/128)*272 + (k%128)*2.  Values
// at k >= K are zero (the device stream is zero there too).
// ---------------------------------------------------------------------------------
__host__ __device__ inline int x_row_stride(int nsl) {
  int rs = nsl * kSliceBytes;
  if (((rs >> 4) & 1) == 0) rs += 16;  // odd number of 16-byte units: batch rows spread
  return rs;
}

// x is read in chunks of 8 consecutive values (16 bytes), XP per thread (4 or 8, chosen by
// the host so that a slice's x fits whenever it can) ahead of the slice's first weight
// loads.  Chunks past the preload are requested after the first weight unit, and loads
// return in order, so they wait for its weights.
constexpr int kXPre = 4;  // the rotation's x preload: 256-value sub-blocks per wave
template <int XP>
struct XPre {
  u32x4 v[XP];
};

// Chunk t of a slice is batch row b = t / per_row, values k0 + 8 (t - b per_row) ...;
// thread j NT + threadIdx.x of an NT-thread workgroup takes chunk t in step j.  per_row is a
// multiple of 64, so the 64 chunks of one wave's step share a row: row_of_wave(tw) (tw = the
// wave's first chunk of the step) runs once per wave, on the scalar unit, and with ONE_ROW
// (batch 1, one slice) the row is 0.  Reads go through a buffer resource over x (B K 2
// bytes): a chunk past K gets an out-of-range offset and reads zeros, with no branch per lane
// and no 64-bit address arithmetic (with ONE_ROW the resource's own size does it).  The 16
// waves of a CU share their SIMDs and scalar unit, and this is the last step before the
// first weight request.
template <int NT, int XP, bool ONE_ROW, typename RowOf>
__device__ __forceinline__ void x_preload(XPre<XP>& xp, rsrc_t xrs, int K, int k0, int per_row,
                                          int nchunks, RowOf row_of_wave, int wave, int tid) {
#pragma unroll
  for (int j = 0; j < XP; ++j) {
    const int tw = wave * 64 + j * NT;
    if (tw < nchunks) {
      const int b = ONE_ROW ? 0 : row_of_wave(tw);
      const int k = k0 + (tid + j * NT - b * per_row) * 8;
      const unsigned off = ONE_ROW || k < K ? (unsigned)(b * K + k) * 2u : kXOutOfRange;
      xp.v[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0));
    }
  }
}

// Plain staging: chunk t lands in its 128-value group of the slice layout.  Chunks past the
// preload are read here, the same way.
template <int NT, int XP, bool ONE_ROW, typename RowOf>
__device__ void stage_plain(uint8_t* lds, const XPre<XP>& xp, rsrc_t xrs, int K, int B, int k0,
                            int nsl, int RS, RowOf row_of_wave, int wave, int tid) {
  const int per_row = nsl * 16;
  const int n = B * per_row;
  auto put = [&](int b, int t, const u32x4& v) {
    const int c8 = t - b * per_row;
    *reinterpret_cast<u32x4*>(lds + b * RS + (c8 >> 4) * kSliceBytes + (c8 & 15) * 16) = v;
  };
#pragma unroll
  for (int j = 0; j < XP; ++j) {
    const int tw = wave * 64 + j * NT;
    if (tw < n) put(ONE_ROW ? 0 : row_of_wave(tw), tid + j * NT, xp.v[j]);
  }
  for (int j = XP; wave * 64 + j * NT < n; ++j) {
    const int b = ONE_ROW ? 0 : row_of_wave(wave * 64 + j * NT);
    const int t = tid + j * NT;
    const int k = k0 + (t - b * per_row) * 8;
    const unsigned off = ONE_ROW || k < K ? (unsigned)(b * K + k) * 2u : kXOutOfRange;
    put(b, t, __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0)));
  }
}

// ---------------------------------------------------------------------------------
// Phase timestamps, compiled in only for the diagnostic library (FB_PHASE_TRACE,
// libfourbit_trace.so): lane i of each wave keeps the s_memrealtime value (a 100 MHz
// clock common to the chip) at which the wave passed phase i; at the end of the kernel each
// wave writes its 64 values to the buffer given to fb_phase_trace_set, at
// (((blockIdx.y * gridDim.x + blockIdx.x) * NW + wave) * 64 + lane).  Lane 16 holds the XCC
// (XCD) id and lane 17 the slice count.  Each mark waits for the wave's outstanding LDS and scalar operations (the
// counter read goes through the scalar memory path), so traced timings run a little long.
// ---------------------------------------------------------------------------------
enum {
  kPhStart = 0, kPhXIssued = 1, kPhXArrived = 2, kPhU0Issued = 3, kPhStages07 = 4,
  kPhPhaseBar = 5, kPhStages811 = 6, kPhStaged = 7, kPhUnit0 = 8, kPhLoopEnd = 9,
  kPhFinalBar = 10, kPhEnd = 11, kPhStaged1 = 12, kPhStaged2 = 13, kPhSliceEnd0 = 14,
  kPhSliceEnd1 = 15, kPhXcc = 16, kPhSlices = 17, kPhGroupLoaded = 18, kPhDecodedAhead = 19
};
#ifdef FB_PHASE_TRACE
struct Phases {
  unsigned lo = 0, hi = 0;
  __device__ __forceinline__ void put(int i, unsigned long long t) {
    const bool me = (int)(threadIdx.x & 63) == i;
    lo = me ? (unsigned)t : lo;
    hi = me ? (unsigned)(t >> 32) : hi;
  }
  __device__ __forceinline__ void mark(int i) { put(i, __builtin_amdgcn_s_memrealtime()); }
  __device__ __forceinline__ void flush(int nw, unsigned long long* buf) {
    put(kPhXcc, __builtin_amdgcn_s_getreg(20 | (15 << 11)));  // HW_REG_XCC_ID
    const size_t wg = (size_t)blockIdx.y * gridDim.x + blockIdx.x;  // split-K: part-major
    const size_t i = (wg * nw + (threadIdx.x >> 6)) * 64 + (threadIdx.x & 63);
    if (buf) buf[i] = ((unsigned long long)hi << 32) | lo;
  }
};
}  // namespace
// Host side: the buffer the next launches write to (fb_phase_trace_set), and its size; one
// copy for both units of the diagnostic library.
namespace fb_trace {
#ifdef FB_GEMV_ILP_TU
extern unsigned long long* g_phase_host;
extern size_t g_phase_entries;
#else
__attribute__((visibility("hidden"))) unsigned long long* g_phase_host = nullptr;
__attribute__((visibility("hidden"))) size_t g_phase_entries = 0;
#endif
}  // namespace fb_trace
using fb_trace::g_phase_entries;
using fb_trace::g_phase_host;
namespace {
// The marks are macros so that the product build's code is exactly what it is without them.
#define PH_DECL Phases ph;
#define PH_PARAM , Phases& ph
#define PH_ARG , ph
#define PH_MARK(i) ph.mark(i)
#define PH_PUT(i, v) ph.put(i, v)
#define PH_FLUSH(nw) ph.flush(nw, phase_buf)
#define PH_KPARAM , unsigned long long* __restrict__ phase_buf
#define PH_KARG(n) , (g_phase_entries >= (size_t)(n) ? g_phase_host : nullptr)
#else
#define PH_DECL
#define PH_PARAM
#define PH_ARG
#define PH_MARK(i) ((void)0)
#define PH_PUT(i, v) ((void)0)
#define PH_FLUSH(nw) ((void)0)
#define PH_KPARAM
#define PH_KARG(n)
#endif

// Blockwise normalised FWHT (fp32 butterflies) of x[b, k0 : k0+kw] into the staged
// layout (rounded to fp16); kw is a whole number of blocks of fb.
//  - Stages 0..7 run in registers.  The B*kw values are cut into 256-value sub-blocks,
//    taken by the NW waves in turn (sub-block i by wave i % NW); lane l holds values
//    4l..4l+3: stages 0-1 are in-lane, stages 2-7 pair lanes l and l ^ 2^(s-2) (lane_xor).
//    The x of a wave's first kXPre sub-blocks is loaded by rot_preload before the slice's
//    weight loads are issued.
//  - Blocks larger than 256 go through LDS (F: B*kw floats) once: each block is read back
//    in 4 groups of 64 positions, taken by the waves in turn; lane l of group c holds value
//    64c + l of each of the block's nb = fb / 256 sub-blocks, so stages 8 .. lg_fb-1 are
//    in-lane butterflies across sub-blocks.
//  - A lane-pair butterfly is one fma: v' = s v + o with o the partner's value and
//    s = +1 in the lower lane (v + o), -1 in the upper one (o - v), the same roundings as
//    the add and the subtract.
// Staged positions k >= kw (up to the slice width) are zero.
struct XRot {
  uint2 v[kXPre];
};

// Each wave loads its first kXPre sub-blocks through a buffer resource over x; a sub-block
// past the last one, and lanes past kw, get an out-of-range offset, which returns zeros and
// moves no data.  The loads are issued back to back with no branch, and nothing waits for
// them before stage_fwht.
// Position of lane l's four values inside a 256-value sub-block: 4l for the butterflies;
// 16 (l % 16) + 4 (l / 16) for the matrix-core transform (blocks of 256 or more), where they
// are row l % 16, columns 4 (l / 16) .. + 3 of the sub-block as a 16 x 16 matrix.
__device__ __forceinline__ int rot_lane_pos(int lane, int fb) {
  return fb >= 256 ? 16 * (lane & 15) + 4 * (lane >> 4) : 4 * lane;
}

template <int NW>
__device__ __forceinline__ void rot_preload(XRot& xr, rsrc_t xrs, int K, int B, int k0, int kw,
                                            int fb, int tid) {
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int nsb = (kw + 255) >> 8;
  const int lpos = rot_lane_pos(lane, fb);
#pragma unroll
  for (int i = 0; i < kXPre; ++i) {
    const int sb = wave + i * NW;  // flat sub-block index over (row, sub-block), uniform
    const int b = B == 1 ? 0 : small_div(sb, nsb);
    const int k = (sb - b * nsb) * 256 + lpos;
    const unsigned off = sb < B * nsb && k < kw ? (unsigned)(b * K + k0 + k) * 2u : kXOutOfRange;
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(xrs, off, 0, 0);
    xr.v[i] = uint2{(unsigned)v[0], (unsigned)v[1]};
  }
}

// v of lane ^ m for a compile-time m (after unrolling), on the VALU for m <= 8: m = 1, 2 by a
// DPP quad permute; m = 4 by a half-row mirror (l ^ 7) then a quad reversal (^ 3); m = 8 by a
// row mirror (l ^ 15) then a half-row mirror (^ 7).  m = 16 by ds_swizzle (xor within 32
// lanes); m = 32 by ds_bpermute.  (gfx950's v_permlane16_swap / v_permlane32_swap with a
// select, all on the VALU, were measured 0.13-0.16 us slower on the 4096-wide rotated layers.)
__device__ __forceinline__ float lane_xor(float v, int m, int lane) {
  const int iv = __builtin_bit_cast(int, v);
  int r;
  if (m == 1) {
    r = __builtin_amdgcn_update_dpp(0, iv, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  } else if (m == 2) {
    r = __builtin_amdgcn_update_dpp(0, iv, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  } else if (m == 4) {
    r = __builtin_amdgcn_update_dpp(0, iv, 0x141, 0xF, 0xF, false);  // row_half_mirror
    r = __builtin_amdgcn_update_dpp(0, r, 0x1B, 0xF, 0xF, false);    // quad_perm [3,2,1,0]
  } else if (m == 8) {
    r = __builtin_amdgcn_update_dpp(0, iv, 0x140, 0xF, 0xF, false);  // row_mirror
    r = __builtin_amdgcn_update_dpp(0, r, 0x141, 0xF, 0xF, false);   // row_half_mirror
  } else if (m == 16) {
    r = __builtin_amdgcn_ds_swizzle(iv, 0x401F);  // bitmask mode: xor 16 within 32 lanes
  } else {
    r = __builtin_amdgcn_ds_bpermute((lane ^ m) << 2, iv);
  }
  return __builtin_bit_cast(float, r);
}

// Position of value p in the fp32 rotation scratch: 16 floats of padding after every 1024,
// so the four 1024-apart lane groups of a phase-2 read fall in different banks.
__host__ __device__ __forceinline__ int fpad(int p) { return p + (p >> 10) * 16; }

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef short bf16x4_t __attribute__((ext_vector_type(4)));

// H16 operand values of lane l: H16[4 (l / 16) + r][l % 16] = (-1)^popcount(.. & ..), as fp16
// (for the first product) and as bf16 (for the second).
struct H16Ops {
  half4_t f;
  bf16x4_t b;
};
__device__ __forceinline__ H16Ops h16_ops(int lane) {
  H16Ops h;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const bool neg = __builtin_popcount((4 * (lane >> 4) + r) & (lane & 15)) & 1;
    h.f[r] = neg ? (_Float16)-1.0f : (_Float16)1.0f;
    h.b[r] = neg ? (short)0xBF80 : (short)0x3F80;
  }
  return h;
}

// Unnormalised 256-point Walsh-Hadamard transform of one sub-block on the matrix cores.  The
// sub-block is a 16 x 16 matrix X (value 16 i + j at row i, column j); H256 x = H16 X H16.
//  1. D1 = X H16: X is the A operand as loaded (lane l: row l % 16, columns 4 (l / 16) ..),
//     fp16 values times +-1 summed in fp32.
//  2. The accumulator of D1 fed back as an A operand is D1 transposed, so D2 = D1^T H16 =
//     (H16 X H16)^T, which lands in lane l as the values 16 (l % 16) + 4 (l / 16) + r: the
//     positions the lane loaded.  D1 goes in as bf16 hi + lo (hi = bf16(d), lo = bf16(d - hi),
//     together within 2^-18 of d), two bf16 products summed in fp32.
__device__ __forceinline__ f32x4 fwht256_mfma(uint2 raw, const H16Ops& h) {
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  const f32x4 d1 =
      __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4_t, raw), h.f, zero, 0, 0, 0);
  bf16x4_t hi, lo;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const __bf16 a = (__bf16)d1[r];
    hi[r] = __builtin_bit_cast(short, a);
    lo[r] = __builtin_bit_cast(short, (__bf16)(d1[r] - (float)a));
  }
  f32x4 d2 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(hi, h.b, zero, 0, 0, 0);
  d2 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(lo, h.b, d2, 0, 0, 0);
  return d2;
}

// A barrier among the first n waves of a workgroup through an LDS counter (zero before the
// first of them arrives), for when the other waves must not wait with them.  The release
// orders each wave's earlier LDS writes before its count; the wait polls with a sleep and is
// bounded, though every one of the n waves arrives.
__device__ __forceinline__ void lds_barrier(int* cnt, int n) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  if ((threadIdx.x & 63) == 0)
    __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  for (int i = 0; i < (1 << 22); ++i) {
    const int v = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (__builtin_amdgcn_readfirstlane(v) >= n) break;
    __builtin_amdgcn_s_sleep(1);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// NW: the waves that take part (the first NW of the workgroup).  LBAR: they meet at the
// LDS barrier on *rbar instead of the workgroup barrier, so the workgroup's other waves are
// free meanwhile.  PRE: every sub-block a wave rotates is among its kXPre preloaded ones (the
// caller's plan guarantees it), so the rotation issues no load of its own: a load there,
// issued after the first weight unit's, could only be waited for together with those weights,
// and the compiler's waits for it (or for its registers' reuse) held the later stages until
// the weights had arrived.
template <int NW, bool LBAR = false, bool PRE = false>
__device__ void stage_fwht(uint8_t* lds, float* F, const XRot& xr, rsrc_t xrs, int K, int B,
                           int k0, int kw, int nsl, int RS, int fb, float sc,
                           int tid, int* rbar PH_PARAM) {
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int lg_fb = 31 - __builtin_clz(fb);
  const int nsb = (kw + 255) >> 8;  // 256-value sub-blocks per batch row
  auto bfly = [&](float& lo, float& hi) {
    const float a = lo, c = hi;
    lo = a + c;
    hi = a - c;
  };
  // per-stage butterfly signs: +1 in the lower lane of a pair, -1 in the upper one
  float sgn[6];
#pragma unroll
  for (int st = 0; st < 6; ++st) sgn[st] = (lane & (1 << st)) ? -1.0f : 1.0f;
  const bool mfma = lg_fb >= 8;  // uniform: whole 256-value sub-blocks on the matrix cores
  const H16Ops hops = h16_ops(lane);
  const int lpos = rot_lane_pos(lane, fb);
  int i = 0;
  for (int sb = wave; sb < B * nsb; sb += NW, ++i) {
    const int b = B == 1 ? 0 : small_div(sb, nsb);
    const int k = (sb - b * nsb) * 256 + lpos;
    const bool live = k < kw;  // kw is a multiple of 128: whole lanes are in or out
    uint2 raw = {0u, 0u};
    if (PRE || i < kXPre) {
#pragma unroll
      for (int j = 0; j < kXPre; ++j)
        if (j == i) raw = xr.v[j];
    } else {
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(
          xrs, live ? (unsigned)(b * K + k0 + k) * 2u : kXOutOfRange, 0, 0);
      raw = uint2{(unsigned)v[0], (unsigned)v[1]};
    }
    float v[4];
    if (mfma) {
      const f32x4 d = fwht256_mfma(raw, hops);
      v[0] = d[0];
      v[1] = d[1];
      v[2] = d[2];
      v[3] = d[3];
    } else {
      const _Float16* h = reinterpret_cast<const _Float16*>(&raw);
      v[0] = (float)h[0];
      v[1] = (float)h[1];
      v[2] = (float)h[2];
      v[3] = (float)h[3];
      if (lg_fb > 0) {
        bfly(v[0], v[1]);
        bfly(v[2], v[3]);
      }
      if (lg_fb > 1) {
        bfly(v[0], v[2]);
        bfly(v[1], v[3]);
      }
#pragma unroll
      for (int st = 0; st < 6; ++st) {
        if (st + 2 < lg_fb) {  // uniform
#pragma unroll
          for (int e = 0; e < 4; ++e)
            v[e] = __builtin_fmaf(sgn[st], v[e], lane_xor(v[e], 1 << st, lane));
        }
      }
    }
    if (!live) continue;
    if (lg_fb <= 8) {
      // four consecutive values of one 128-group: one 8-byte store
      const half4_t hv = {(_Float16)(v[0] * sc), (_Float16)(v[1] * sc), (_Float16)(v[2] * sc),
                          (_Float16)(v[3] * sc)};
      *reinterpret_cast<half4_t*>(lds + b * RS + (k >> 7) * kSliceBytes + (k & 127) * 2) = hv;
    } else {
      const int p = b * kw + k;
      *reinterpret_cast<f32x4*>(F + fpad(p)) = f32x4{v[0], v[1], v[2], v[3]};
    }
  }
  PH_MARK(kPhStages07);
  if (lg_fb > 8) {
    if constexpr (LBAR)
      lds_barrier(rbar, NW);
    else
      __syncthreads();
    PH_MARK(kPhPhaseBar);
    // Stages 8 .. lg_fb-1 run across the nb = fb / 256 sub-blocks of a block, in registers:
    // a wave takes 64 positions p of one block at a time (lane = p % 64) and holds value p of
    // each of its sub-blocks, so the stages are in-lane butterflies on sub-block index bits
    // 0, 1, 2, 3 in turn.  kw is a whole number of blocks (fb divides K, and a K-slice holds
    // whole blocks).
    const int bpr = kw >> lg_fb;  // blocks per batch row
    const int ngroups = B * bpr * 4;
    // NB = fb / 256 sub-blocks per block, fixed at compile time so that the group's loads,
    // butterflies and stores are straight-line code (with a runtime count the compiler
    // branched around each and waited for the LDS after every store)
    auto groups = [&](auto nbc) {
      constexpr int NB = decltype(nbc)::value;
      for (int g = wave; g < ngroups; g += NW) {
        const int blk = g >> 2;  // uniform
        const int p = (g & 3) * 64 + lane;
        const int e0 = blk * fb + p;  // value index of sub-block 0, over the batch
        float v[NB];
#pragma unroll
        for (int j = 0; j < NB; ++j) v[j] = F[fpad(e0 + j * 256)];
#pragma unroll
        for (int t = 0; (1 << t) < NB; ++t) {
#pragma unroll
          for (int j = 0; j < NB; ++j)
            if (!(j & (1 << t))) bfly(v[j], v[j | (1 << t)]);
        }
        if (g == wave) PH_MARK(kPhGroupLoaded);
        const int bb = B == 1 ? 0 : small_div(blk, bpr);  // batch row (uniform)
        const int k0b = (blk - bb * bpr) * fb + p;         // k of sub-block 0 within the row
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const int k = k0b + j * 256;
          *(reinterpret_cast<_Float16*>(lds + bb * RS + (k >> 7) * kSliceBytes) + (k & 127)) =
              (_Float16)(v[j] * sc);
        }
      }
    };
    if (lg_fb == 12)
      groups(std::integral_constant<int, 16>());
    else if (lg_fb == 11)
      groups(std::integral_constant<int, 8>());
    else if (lg_fb == 10)
      groups(std::integral_constant<int, 4>());
    else
      groups(std::integral_constant<int, 2>());
  }
  PH_MARK(kPhStages811);
  // zeros past the rotated width (the weight stream is zero there too)
  const int width = nsl * 128;
  for (int t = tid; t < B * ((width - kw) >> 3); t += NW * 64) {
    const int b = t / ((width - kw) >> 3);
    const int k = kw + (t - b * ((width - kw) >> 3)) * 8;
    *reinterpret_cast<u32x4*>(lds + b * RS + (k >> 7) * kSliceBytes + (k & 127) * 2) =
        u32x4{0u, 0u, 0u, 0u};
  }
}

__host__ __device__ inline int x_lds_bytes(int B, int K, int SPL, int fwht_block) {
  int b = B * x_row_stride(SPL * 4);
  if (fwht_block > 256) b += fpad(B * min(K, SPL * 512)) * 4 + 64;  // fp32 scratch of the rotation
  return (b + 15) & ~15;
}

// A unit decoded ahead of its x: the 16 A operands of its MFMAs, in unit_partial's order.
struct Dec {
  u32x4 a[16];
};
template <int FMT, int XDT>
__device__ __forceinline__ void unit_decode(const Rec<FMT>& r, Dec& D) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float scale = 1.0f;
    if constexpr (FMT == FB_FMT_E2M1)
      scale = __builtin_bit_cast(float, ((r.t0.x >> (8 * c)) & 0xFFu) << 23);
#pragma unroll
    for (int d = 0; d < 4; d += 2) {
      if constexpr (FMT == FB_FMT_GF4) {
        gf4_decode16(r.nib[c][d], r.nib[c][d + 1], r.t0, r.t1, D.a[c * 4 + d], D.a[c * 4 + d + 1]);
      } else {
        D.a[c * 4 + d] = e2m1_decode8<XDT>(r.nib[c][d], scale);
        D.a[c * 4 + d + 1] = e2m1_decode8<XDT>(r.nib[c][d + 1], scale);
      }
    }
  }
}
// The MFMAs of a decoded unit: the same products, accumulated in the same order, as
// unit_partial's, so the same bits.
template <int XDT>
__device__ __forceinline__ f32x4 unit_mfma(const Dec& D, const uint8_t* xs) {
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < 4; ++c) {
#pragma unroll
    for (int d = 0; d < 4; d += 2) {
      const u32x4 xv0 = *reinterpret_cast<const u32x4*>(xs + (c * 32 + d * 8) * 2);
      const u32x4 xv1 = *reinterpret_cast<const u32x4*>(xs + (c * 32 + d * 8 + 8) * 2);
      acc0 = mfma<XDT>(D.a[c * 4 + d], xv0, acc0);
      acc1 = mfma<XDT>(D.a[c * 4 + d + 1], xv1, acc1);
    }
  }
  return acc0 + acc1;
}

// Decode + MFMA of one unit held in registers: the lane's f32x4 of partial sums (rows
// 4q..4q+3 of the tile, batch column L % 16).  xs: the unit's x in the staged layout.
template <int FMT, int XDT>
__device__ __forceinline__ f32x4 unit_partial(const Rec<FMT>& r, const uint8_t* xs) {
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float scale = 1.0f;
    if constexpr (FMT == FB_FMT_E2M1)
      scale = __builtin_bit_cast(float, ((r.t0.x >> (8 * c)) & 0xFFu) << 23);
#pragma unroll
    for (int d = 0; d < 4; d += 2) {
      u32x4 a0, a1;
      if constexpr (FMT == FB_FMT_GF4) {
        gf4_decode16(r.nib[c][d], r.nib[c][d + 1], r.t0, r.t1, a0, a1);
      } else {
        a0 = e2m1_decode8<XDT>(r.nib[c][d], scale);
        a1 = e2m1_decode8<XDT>(r.nib[c][d + 1], scale);
      }
      const u32x4 xv0 = *reinterpret_cast<const u32x4*>(xs + (c * 32 + d * 8) * 2);
      const u32x4 xv1 = *reinterpret_cast<const u32x4*>(xs + (c * 32 + d * 8 + 8) * 2);
      acc0 = mfma<XDT>(a0, xv0, acc0);
      acc1 = mfma<XDT>(a1, xv1, acc1);
    }
  }
  return acc0 + acc1;
}

// ---------------------------------------------------------------------------------
// The native FP4 path (fb_gemv_mx): E2M1 weights times x split into two MX-E4M3 terms
// ---------------------------------------------------------------------------------
// v_mfma_scale_f32_16x16x128_f8f6f4 multiplies the E2M1 codes as they are stored, with their
// E8M0 group scales, by an 8-bit B operand with E8M0 scales of its own per 32 K-values.  x
// (bf16) is split once per call into x = t0 + t1: t0 rounds x and t1 rounds what t0 left,
// each to E4M3 values times a power of two 2^e per 32-value block, e the smallest for which
// the block's largest magnitude is at most 448 (E4M3's largest finite value), so no value
// saturates.  A bf16 value has 8 significant bits and an E4M3 value 4, so the two terms hold
// x exactly unless a block spans more than E4M3's exponent range (values 2^14 times or more
// below the block's largest, which then lose low bits).
//
// Layout of the split, which the GEMV stages as it stages bf16 x (2 bytes per value): for
// batch row b and 128-value group g, 256 bytes at (b K/128 + g) 256 -- the 128 E4M3 codes of
// t0, then the 128 of t1, in K order; the scales from byte mx_scale_offset(B, K) on, 8 bytes
// per (b, g) -- the E8M0 bytes of the group's four 32-value blocks for t0, then for t1.  In
// LDS the scales sit in the 16-byte pad of each staged 128-value group.
constexpr int kFmtMx = 2;  // internal format code: E2M1 stream, x as the MX split

__host__ __device__ inline size_t mx_scale_offset(int B, int K) {
  return ((size_t)B * K * 2 + 255) & ~size_t(255);
}
__host__ __device__ inline size_t mx_split_bytes(int B, int K) {
  return mx_scale_offset(B, K) + (((size_t)B * (K / 128) * 8 + 255) & ~size_t(255));
}

// E8M0 byte (e + 127) of a 32-value block whose largest magnitude has the bf16 bit pattern a
// (sign cleared): e is the smallest exponent with that magnitude at most 448 2^e (448 = 1.75 2^8,
// E4M3's largest finite value), and at least -127.  With a = (biased exponent E, fraction F, 7
// bits), e + 127 = E - 8 + (F > 0x60); adding 31 carries into E exactly when F > 0x60.  A zero
// or bf16-subnormal block gets 0 (2^-127).  x must be finite.
__device__ __forceinline__ unsigned mx_scale_byte(unsigned a) {
  const int s = (int)((a + 31u) >> 7) - 8;
  return s < 0 ? 0u : (unsigned)s;
}

// Largest of v over the lane's quad (the 4 threads of one 32-value block), by two DPP quad
// permutes.
__device__ __forceinline__ unsigned quad_max(unsigned v) {
  v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));  // [1,0,3,2]
  v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));  // [2,3,0,1]
  return v;
}

typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
// A word as two bf16 values.  Taken by value: clang's __builtin_bit_cast of a vector element
// (raw.y) reads the vector's first element instead.
__device__ __forceinline__ bf16x2_t bf16_pair(unsigned w) { return __builtin_bit_cast(bf16x2_t, w); }

// The split: one thread per 8 consecutive values (n8 = B K / 8 threads, a multiple of 16), so
// the 4 threads of a 32-value block are one aligned lane quad and a 128-value group's 16
// threads are aligned lanes of one wave.  The rounding is gfx950's scaled conversions:
// v_cvt_scalef32_pk_fp8_{bf16,f32} divide two values by the power of two whose exponent field
// is their f32 scale operand's (all 8 bits: field 0 is 2^-127, as in E8M0) and round to the
// nearest E4M3 value, ties to even, subnormals included, with no saturation needed (every
// quotient is at most 448 by the choice of e); v_cvt_scalef32_pk_f32_fp8 multiplies the codes
// back, exactly wherever the product is within fp32's range (below).  The GPU tests
// hold the result to the oracle's split byte for byte, over every finite bf16 value.
//  - Term 0 rounds x.  Its block maximum is taken on the bf16 bit patterns (magnitudes order
//    as unsigned integers), two at a time.
//  - Term 1 rounds t = x - term 0, computed in fp32 and exact (x and term 0 lie on x's bf16
//    grid, within a factor 2 of each other, or term 0 is zero), and itself a bf16 value, so
//    its maximum's top 16 bits are its bf16 pattern.
__global__ __launch_bounds__(64) void mx_split_kernel(const uint16_t* __restrict__ x,
                                                      uint8_t* __restrict__ out, int n8,
                                                      size_t sc_off) {
  const int i = blockIdx.x * 64 + threadIdx.x;
  const bool in = i < n8;
  const u32x4 raw = in ? *reinterpret_cast<const u32x4*>(x + (size_t)i * 8) : u32x4{0u, 0u, 0u, 0u};
  const size_t rec = (size_t)(i >> 4);  // (b K/128 + g): values 8i.. are b K + k
  uint8_t* codes = out + rec * 256 + (i & 15) * 8;
  uint8_t* sbyte = out + sc_off + rec * 8 + ((i >> 2) & 3);  // the block's scale byte, term 0
  const bool first = in && (i & 3) == 0;                     // the block's first thread writes it

  // term 0
  const u16x2 m01 = __builtin_elementwise_max(__builtin_bit_cast(u16x2, raw.x & 0x7FFF7FFFu),
                                              __builtin_bit_cast(u16x2, raw.y & 0x7FFF7FFFu));
  const u16x2 m23 = __builtin_elementwise_max(__builtin_bit_cast(u16x2, raw.z & 0x7FFF7FFFu),
                                              __builtin_bit_cast(u16x2, raw.w & 0x7FFF7FFFu));
  const u16x2 m = __builtin_elementwise_max(m01, m23);
  const unsigned sb0 = mx_scale_byte(quad_max(max((unsigned)m.x, (unsigned)m.y)));
  const float sc0 = __builtin_bit_cast(float, sb0 << 23);
  s16x2 c01 = {0, 0}, c23 = {0, 0};
  c01 = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(c01, bf16_pair(raw.x), sc0, false);
  c01 = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(c01, bf16_pair(raw.y), sc0, true);
  c23 = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(c23, bf16_pair(raw.z), sc0, false);
  c23 = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(c23, bf16_pair(raw.w), sc0, true);
  const unsigned w0 = __builtin_bit_cast(unsigned, c01), w1 = __builtin_bit_cast(unsigned, c23);
  if (in) *reinterpret_cast<uint2*>(codes) = uint2{w0, w1};
  if (first) sbyte[0] = (uint8_t)sb0;

  // term 1: t = x - term 0
  // A block of scale 2^120 (the largest a finite bf16 block gets) can round to 256 2^120 =
  // 2^128, past fp32's range: there term 0 is taken back at half its value h and t = (x - h) - h,
  // both steps exact (x and h have one sign and lie on x's bf16 grid).
  const bool top = sb0 >= 247;
  const float scq = __builtin_bit_cast(float, (sb0 - (top ? 1u : 0u)) << 23);
  const f32x2 q[4] = {__builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w0, scq, false),
                      __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w0, scq, true),
                      __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w1, scq, false),
                      __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w1, scq, true)};
  float t[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    t[2 * j] = __builtin_bit_cast(float, raw[j] << 16) - q[j].x;
    t[2 * j + 1] = __builtin_bit_cast(float, raw[j] & 0xFFFF0000u) - q[j].y;
  }
  if (top) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      t[2 * j] -= q[j].x;
      t[2 * j + 1] -= q[j].y;
    }
  }
  float a = __builtin_fmaxf(__builtin_fabsf(t[0]), __builtin_fabsf(t[1]));
#pragma unroll
  for (int j = 2; j < 8; ++j) a = __builtin_fmaxf(a, __builtin_fabsf(t[j]));
  const unsigned sb1 = mx_scale_byte(quad_max(__builtin_bit_cast(unsigned, a) >> 16));
  const float sc1 = __builtin_bit_cast(float, sb1 << 23);
  s16x2 d01 = {0, 0}, d23 = {0, 0};
  d01 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(d01, t[0], t[1], sc1, false);
  d01 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(d01, t[2], t[3], sc1, true);
  d23 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(d23, t[4], t[5], sc1, false);
  d23 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(d23, t[6], t[7], sc1, true);
  if (in)
    *reinterpret_cast<uint2*>(codes + 128) =
        uint2{__builtin_bit_cast(unsigned, d01), __builtin_bit_cast(unsigned, d23)};
  if (first) sbyte[4] = (uint8_t)sb1;
}

typedef int i32x8 __attribute__((ext_vector_type(8)));
template <int C>
__device__ __forceinline__ f32x4 mfma_mx(const u32x4& a, const u32x4& b0, const u32x4& b1,
                                         const f32x4& acc, unsigned sa, unsigned sb) {
  const i32x8 av = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0};  // fp4: 4 dwords read
  const i32x8 bv = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w,
                    (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
  // A: E2M1 (cbsz 4), B: E4M3 (blgp 0); byte C of each lane's scale word
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, acc, 4, 0, C, (int)sa, C,
                                                          (int)sb);
}

// One unit on the FP4 MFMA, 8 MFMAs (4 chunks x 2 terms).  Lane L = n + 16 q gives chunk c
// of its item q as A (32 codes; scale byte c of its record) -- K-block q of the MFMA.  The
// MFMA pairs value 16 h + j (j < 16) of K-block g with B byte 16 (g >> 1) + j of B lane
// group 2 (g & 1) + h, and takes block g's B scale from lane n + 16 g (found by one-hot
// probes of the instruction on gfx950).  So B lane (n, q) holds values 16 (q & 1) .. +15 of
// chunk c of items q >> 1 and 2 + (q >> 1), and the scale of its own item's block c.
// xs: the span's first staged group of batch row n.
// B operands of chunk C: terms 0 and 1, each 16 bytes from two groups.
struct MxB {
  u32x4 t0a, t0b, t1a, t1b;
};
template <int C>
__device__ __forceinline__ void mx_read(const uint8_t* d, MxB& b) {
  b.t0a = *reinterpret_cast<const u32x4*>(d + C * 32);
  b.t0b = *reinterpret_cast<const u32x4*>(d + 2 * kSliceBytes + C * 32);
  b.t1a = *reinterpret_cast<const u32x4*>(d + 128 + C * 32);
  b.t1b = *reinterpret_cast<const u32x4*>(d + 2 * kSliceBytes + 128 + C * 32);
}
// Chunk C's two MFMAs, with chunk C + 1's reads issued first (two buffers of 16 registers
// instead of all 64 up front, which left the sliced kernels spilling).
template <int C>
__device__ __forceinline__ void mx_step(const Rec<kFmtMx>& r, const uint8_t* d, uint2 sx,
                                        MxB (&b)[2], f32x4& acc0, f32x4& acc1) {
  if constexpr (C < 3) mx_read<C + 1>(d, b[(C + 1) & 1]);
  acc0 = mfma_mx<C>(r.nib[C], b[C & 1].t0a, b[C & 1].t0b, acc0, r.t0.x, sx.x);
  acc1 = mfma_mx<C>(r.nib[C], b[C & 1].t1a, b[C & 1].t1b, acc1, r.t0.x, sx.y);
  // keeps the MFMAs here: otherwise they sink into the slot write's per-lane branch, after
  // every read of the unit
  asm volatile("" : "+v"(acc0), "+v"(acc1));
  __builtin_amdgcn_sched_barrier(0);
}
__device__ __forceinline__ f32x4 unit_partial_mx(const Rec<kFmtMx>& r, const uint8_t* xs, int q) {
  const uint8_t* d = xs + (q >> 1) * kSliceBytes + (q & 1) * 16;
  const uint2 sx = *reinterpret_cast<const uint2*>(xs + q * kSliceBytes + 256);
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  MxB b[2];
  mx_read<0>(d, b[0]);
  __builtin_amdgcn_sched_barrier(0);
  mx_step<0>(r, d, sx, b, acc0, acc1);
  mx_step<1>(r, d, sx, b, acc0, acc1);
  mx_step<2>(r, d, sx, b, acc0, acc1);
  mx_step<3>(r, d, sx, b, acc0, acc1);
  return acc0 + acc1;
}
// LDS of the zero block that MFMA columns past the batch read: the MX unit reads up to
// 3 groups + 256 + 8 bytes past its span base.
constexpr int zero_bytes(int fmt) { return fmt == kFmtMx ? 1088 : 256; }

// ---------------------------------------------------------------------------------
// The GEMV kernel
// ---------------------------------------------------------------------------------
// The first 15 argument dwords arrive preloaded in SGPRs and hold everything but the
// output; y, N and ydt come through a scalar load that completes long before the epilogue
// needs them (the LDS size of staged x is derived in the kernel, and the rotation scale is
// an argument, so nothing early waits for that load).  tq, tr: row tiles per workgroup = tq (+1 for the
// first tr workgroups); GS: 512-element spans per row; RS: LDS bytes per staged x row;
// spl_m: div_magic(SPL).
// MODE: kFlat = one K-slice, no rotation (the common case); kFlat1 = the same at batch 1;
// kSliced = several K-slices, no rotation; kRotated = rotation of x; kRot1 = rotation at
// batch 1 in one K-slice; kSplitK = one K-part per workgroup (blockIdx.y = the part), the
// parts' fp32 sums written to the caller's workspace and added by splitk_sum; kRotDA = kRot1
// with decode-ahead waves: the first half of the workgroup's waves rotate x (meeting at an LDS
// barrier of their own), while the second half load and decode their first unit into
// registers, so that this decode runs during the rotation's waits instead of after it.  Each is
// compiled with only the staging it needs, which keeps the kernel short and its registers
// few.
// kRotDAall = kRotDA where a workgroup owns no more units than waves: the rotating waves also
// decode their one unit before the staging barrier (with more units that would hold the
// barrier back).
// kSpanX = batch 2-16 without K-slices: wave w owns spans w, w + NW, ... of every row tile of
// the workgroup and stages each span's x in an LDS region of its own (XP is then the most row
// tiles a workgroup owns, whose sums the wave keeps in registers).
enum { kFlat = 0, kSliced = 1, kRotated = 2, kRot1 = 3, kFlat1 = 4, kSplitK = 5, kRotDA = 6,
       kRotDAall = 7, kSpanX = 8 };
// NW: waves per workgroup.  16 (one workgroup per CU) in general; 8 (two per CU) for
// layers with few row tiles per CU, where twice the workgroups, each with half the waves,
// finish sooner.
template <int FMT, int XDT, int MODE, int NW, int XP>
__global__ __launch_bounds__(NW * 64) void gemv_kernel(
    const uint8_t* __restrict__ w, const void* __restrict__ x, int K, int Bin, int SPL, int GS,
    int tq, int tr, unsigned spl_m, int S, int fwht_block, int RS, float fwht_scale,
    void* __restrict__ y, int N, int ydt PH_KPARAM) {
  extern __shared__ __align__(16) uint8_t lds[];
  PH_DECL
  PH_MARK(kPhStart);
  // kRot1 / kFlat1: batch 1 in one K-slice, with both fixed at compile time so that the
  // batch-row and slice bookkeeping folds away (16 waves per CU share one scalar unit, and
  // the prologue is on the critical path of small layers)
  constexpr bool da_all = MODE == kRotDAall;
  constexpr bool da = MODE == kRotDA || da_all;
  constexpr bool rot1 = MODE == kRot1 || da;
  constexpr bool flat1 = MODE == kFlat1;
  constexpr int NWR = da ? NW / 2 : NW;  // waves that rotate x
  const int B = rot1 || flat1 ? 1 : Bin;
  // batch 1 in one K-slice: each tile is reduced by the wave that finishes it
  constexpr bool tile_reduce = rot1 || flat1;
  const int nslices = MODE == kFlat || rot1 || flat1 ? 1 : S;
  // kSplitK: this workgroup runs the one slice (K-part) blockIdx.y of the sliced layout and
  // writes its part's sums, fp32, to y + part * B * N
  constexpr bool splitk = MODE == kSplitK;
  const int s_begin = splitk ? (int)blockIdx.y : 0;
  const int s_end = splitk ? s_begin + 1 : nslices;
  void* yo = splitk ? static_cast<void*>(static_cast<float*>(y) + (size_t)s_begin * Bin * N) : y;
  const int xbytes = x_lds_bytes(B, K, SPL, fwht_block);  // staged x; the slots follow
  constexpr int BB = FMT == FB_FMT_GF4 ? fb::kGf4BlockBytes : fb::kE2m1BlockBytes;
  constexpr int NT = NW * 64;
  const int g = blockIdx.x;
  const int t0 = g * tq + min(g, tr);
  const int t1 = t0 + tq + (g < tr ? 1 : 0);
  const int nsl = SPL * 4;
  // Unit u of a slice is span u % sp of tile t0 + u / sp, with sp = SPL spans per slice;
  // the last K-slice may hold fewer (spl_last), and then has fewer units.  A unit's slot
  // is tile * SPL + span in every slice.
  const int spl_last = GS - (S - 1) * SPL;
  int sp = SPL;
  unsigned sp_m = spl_m;
  int nu = (t1 - t0) * SPL;  // units of this workgroup in the current slice
  auto tile_of = [&](int u) { return fdiv(u, sp, sp_m); };
  // LDS: unit counter (16 B) | zero block (256 B) | staged x (xbytes) | partial-sum slots |
  // per-tile unit counts
  int* counter = reinterpret_cast<int*>(lds);
  uint8_t* zeros = lds + 16;
  uint8_t* xst = lds + 16 + zero_bytes(FMT);
  f32x4* slots = reinterpret_cast<f32x4*>(xst + xbytes);


  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: SGPR math
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;  // batch column / row within tile
  const int q = lane >> 4;    // K-quarter of the span / output row group
  // MFMA columns >= B multiply zeros (read from one 256-byte block whatever the span):
  // their results are not used, and zeros keep the matrix core from switching.
  constexpr bool mx = FMT == kFmtMx;  // the native FP4 path reads 3 groups from the span base
  const uint8_t* xl = col < B ? xst + col * RS + (mx ? 0 : q * kSliceBytes) : zeros;
  const int xspan = col < B ? 4 * kSliceBytes : 0;  // x bytes per span for this lane

  // After two fixed units per wave, the waves take units from the workgroup's LDS counter, so a wave that the SIMD's
  // issue order favours does more of them and all waves finish together.
  // lane 0 holds the fetched index; it is made uniform when it is used, a step later, so
  // the atomic's latency is hidden.
  auto grab = [&]() -> int {
    int u = 0;
    if (lane == 0)
      u = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    return u;
  };
  // Offsets are taken from this workgroup's first block, so a unit's offset stays below
  // 2^31 (the host checks that a workgroup's blocks span less) whatever the layer's size.
  const uint8_t* wbase = w + (int64_t)t0 * GS * BB;
  auto unit_off = [&](int s, int u) -> unsigned {
    const int lt = tile_of(u);
    return (unsigned)((lt * GS + s * SPL + (u - lt * sp)) * BB);
  };

  // Per-tile count of the last slice's finished units, after the slots.
  int* tile_cnt = reinterpret_cast<int*>(slots + (size_t)(t1 - t0) * SPL * 4 * B);
  // y of tile lt: each output sums its tile's span slots in span order (the wave that
  // finished the tile's last unit does it, while the others go on).
  auto reduce_tile = [&](int lt) {
    for (int o = lane; o < 16 * B; o += 64) {
      const int r = o & 15, c = o >> 4;
      const int row = (t0 + lt) * 16 + r;
      const f32x4* sl = slots + ((size_t)lt * SPL * 4 + (r >> 2)) * B + c;
      float sum = 0.0f;
      for (int j = 0; j < SPL; ++j) sum += sl[(size_t)j * 4 * B][r & 3];
      if (row < N) store_y(yo, (int64_t)c * N + row, sum, ydt);
    }
  };
  // Decode + MFMA of unit u (slice s) from record r; the unit's partial sums go to its own
  // LDS slot (added to the earlier slices' value), so the final sum has a fixed order
  // whichever wave did the unit.  At batch 1 (kFlat1, kRot1) the unit is counted on its
  // tile, and the unit that completes a tile reduces it: a tile is 16 outputs, and the
  // workgroup then needs no final barrier and epilogue.  Larger batches keep the epilogue,
  // spread over all the workgroup's threads (16 B outputs per tile for one wave was slower).
  auto finish = [&](const f32x4& acc, int s, int lt, int span) {
    if (col < B) {
      f32x4* sl = slots + ((size_t)(lt * SPL + span) * 4 + q) * B + col;
      if (s == s_begin)
        *sl = acc;
      else
        *sl += acc;
    }
    if constexpr (tile_reduce) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");  // the slot, then the count
      int old = 0;
      if (lane == 0)
        old = __hip_atomic_fetch_add(&tile_cnt[lt], 1, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_WORKGROUP);
      if (__builtin_amdgcn_readfirstlane(old) + 1 == sp) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");  // every slot of lt
        reduce_tile(lt);
      }
    }
  };
  auto process = [&](const Rec<FMT>& r, int s, int u) {
    const int lt = tile_of(u);
    const int span = u - lt * sp;
    f32x4 acc;
    if constexpr (mx)
      acc = unit_partial_mx(r, xl + span * xspan, q);
    else
      acc = unit_partial<FMT, XDT>(r, xl + span * xspan);
    finish(acc, s, lt, span);
  };

  // Two record buffers: the loads of the next unit are in flight while one is decoded.
  // Loads past the last unit use the empty resource (no branch, no traffic).  Unit
  // indices only grow, so the first index past the end stops the wave.
  Rec<FMT> ring[2];
  auto issue = [&](int s, int u, Rec<FMT>& r) {
    const bool real = u < nu;  // wave-uniform: only the range changes
    const rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(wbase), (short)0,
                                                        real ? 0x7fffffff : 0, kRsrcWord3);
    load_rec<FMT>(rs, real ? unit_off(s, u) : 0u, lane, r);
  };
  // x through a buffer resource (out-of-range offsets read zeros)
  const rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(x), (short)0, B * K * 2,
                                                       kRsrcWord3);
  // MX path: the split's block scales, 8 bytes per (batch row, 128-value group), staged into
  // the pad of each staged group (zeros past K).  Entry i of a slice is row i / nsl, group
  // k0 / 128 + i % nsl.  They follow the codes in the split's layout, so no argument is
  // needed for them.
  const int G = K / 128;
  const uint8_t* xsc = static_cast<const uint8_t*>(x) + mx_scale_offset(Bin, K);
  const rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(xsc), (short)0,
                                                       mx ? B * G * 8 : 0, kRsrcWord3);
  auto sc_load = [&](int i, int k0) -> uint2 {
    const int b = fdiv(i >> 2, SPL, spl_m);  // i / nsl, nsl = 4 SPL
    const int gi = k0 / 128 + i - b * nsl;
    const unsigned off = gi < G ? (unsigned)(b * G + gi) * 8u : kXOutOfRange;
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(srs, off, 0, 0));
  };
  auto sc_store = [&](int i, uint2 v) {
    const int b = fdiv(i >> 2, SPL, spl_m);
    *reinterpret_cast<uint2*>(xst + b * RS + (i - b * nsl) * kSliceBytes + 256) = v;
  };
  if constexpr (MODE == kSpanX) {
    // Each wave owns the spans wave, wave + NW, ... of every row tile of the workgroup and
    // stages the x of one span at a time (B rows of 512 values, RS bytes per row) in an LDS
    // region of its own, so no wave waits for another before the epilogue.  Unit i of the
    // wave is span wave + (i / nt) NW of tile i % nt; the wave adds its units' partial sums
    // per tile in registers, in its span order, and after the last unit writes them to the
    // (tile, wave) slots (over the x regions); each output then adds its tile's NW slots in
    // wave order.
    constexpr int kTMax = XP;  // row tiles per workgroup, at most (the host checks)
    const int nt = t1 - t0;
    uint8_t* xw = xst + wave * B * RS;
    f32x4* wsl = reinterpret_cast<f32x4*>(xst);
    const uint8_t* xlw = col < B ? xw + col * RS + (mx ? 0 : q * kSliceBytes) : zeros;
    const int nsw = wave < GS ? (GS - 1 - wave) / NW + 1 : 0;  // spans of this wave
    const int nuw = nsw * nt;
    // the native FP4 path stages the split's two E4M3 terms where bf16 x would be (the same
    // bytes per value) and the group scales in each group's pad: lane 4 b + g takes batch
    // row b's group g of the span
    u32x4 xv[16];
    uint2 xsv = {0u, 0u};
    auto x_load = [&](int sp0) {
      const int k = sp0 * 512 + lane * 8;
#pragma unroll
      for (int b = 0; b < 16; ++b)
        if (b < B) {
          const unsigned off = k < K ? (unsigned)(b * K + k) * 2u : kXOutOfRange;
          xv[b] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0));
        }
      if constexpr (mx) {
        const int gi = sp0 * 4 + (lane & 3);
        const unsigned off = gi < G ? (unsigned)((lane >> 2) * G + gi) * 8u : kXOutOfRange;
        if ((lane >> 2) < B)
          xsv = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(srs, off, 0, 0));
      }
    };
    auto x_put = [&]() {
      uint8_t* d = xw + (lane >> 4) * kSliceBytes + (lane & 15) * 16;
#pragma unroll
      for (int b = 0; b < 16; ++b)
        if (b < B) *reinterpret_cast<u32x4*>(d + b * RS) = xv[b];
      if constexpr (mx)
        if ((lane >> 2) < B)
          *reinterpret_cast<uint2*>(xw + (lane >> 2) * RS + (lane & 3) * kSliceBytes + 256) = xsv;
    };
    int is = wave, it = 0, ni = 0;  // the next unit to request
    auto w_issue = [&](Rec<FMT>& r) {
      const bool real = ni < nuw;
      const rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(wbase), (short)0,
                                                          real ? 0x7fffffff : 0, kRsrcWord3);
      load_rec<FMT>(rs, real ? (unsigned)((it * GS + is) * BB) : 0u, lane, r);
      ++ni;
      if (++it == nt) {
        it = 0;
        is += NW;
      }
    };
    if (threadIdx.x < zero_bytes(FMT) / 16)
      reinterpret_cast<u32x4*>(zeros)[threadIdx.x] = u32x4{0u, 0u, 0u, 0u};
    // GF4: units finished per wave, after the x regions / slots
    int* prog = reinterpret_cast<int*>(xst + max(NW * B * RS, nt * NW * B * 64));
    if constexpr (FMT == FB_FMT_GF4)
      if (threadIdx.x < NW) prog[threadIdx.x] = 0;
    int done = 0;
    if (nsw) x_load(wave);
    PH_MARK(kPhXIssued);
    Rec<FMT> rg[2];
    w_issue(rg[0]);
    PH_MARK(kPhU0Issued);
    __syncthreads();  // the zero block
    f32x4 acc[kTMax];
    int sc = wave, lt = 0;
    auto step = [&](const Rec<FMT>& cur, Rec<FMT>& nxt) {
      // GF4 (whose decode keeps the SIMDs busy): waves w and w + 4 share a SIMD, which issues
      // the older one first; the one that has finished fewer units takes the higher priority
      if constexpr (FMT == FB_FMT_GF4) {
        const int pd = __builtin_amdgcn_readfirstlane(
            __hip_atomic_load(prog + (wave ^ 4), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
        if (done < pd)
          __builtin_amdgcn_s_setprio(1);
        else
          __builtin_amdgcn_s_setprio(0);
      }
      if (lt == 0) {
        x_put();
        PH_MARK(sc == wave ? kPhStaged : sc == wave + NW ? kPhStaged1 : kPhStaged2);
        if (sc + NW < GS) x_load(sc + NW);  // in flight during this span's units
      }
      w_issue(nxt);
      __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the compute
      f32x4 p;
      if constexpr (mx)
        p = unit_partial_mx(cur, xlw, q);
      else
        p = unit_partial<FMT, XDT>(cur, xlw);
      const bool first = sc == wave;
      if (first && lt == 0) PH_MARK(kPhUnit0);
      if constexpr (FMT == FB_FMT_GF4) {
        ++done;
        if (lane == 0)
          __hip_atomic_store(prog + wave, done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
#pragma unroll
      for (int t = 0; t < kTMax; ++t)  // lt is wave-uniform: a scalar branch per tile
        if (t == lt) acc[t] = first ? p : acc[t] + p;
      if (++lt == nt) {
        lt = 0;
        sc += NW;
      }
    };
    for (int i = 0; i < nuw; i += 2) {
      step(rg[0], rg[1]);
      if (i + 1 >= nuw) break;
      step(rg[1], rg[0]);
    }
    if constexpr (FMT == FB_FMT_GF4) __builtin_amdgcn_s_setprio(0);
    PH_MARK(kPhLoopEnd);
    __syncthreads();  // every wave is done with its x: the slots may take the x regions
    if (col < B) {  // a wave without spans (GS < NW) adds zeros
#pragma unroll
      for (int t = 0; t < kTMax; ++t)
        if (t < nt)
          wsl[((size_t)(t * NW + wave) * 4 + q) * B + col] = nsw ? acc[t] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    __syncthreads();  // every slot complete
    PH_MARK(kPhFinalBar);
    for (int e = threadIdx.x; e < nt * 256; e += NT) {
      const int c = e & 15;
      if (c >= B) continue;
      const int r = (e >> 4) & 15;
      const int lt2 = e >> 8;
      const int row = (t0 + lt2) * 16 + r;
      const f32x4* sl = wsl + ((size_t)lt2 * NW * 4 + (r >> 2)) * B + c;
      // a fixed count, so the NW reads are issued together before the adds
      float v[NW];
#pragma unroll
      for (int j = 0; j < NW; ++j) v[j] = sl[(size_t)j * 4 * B][r & 3];
      float sum = 0.0f;
#pragma unroll
      for (int j = 0; j < NW; ++j) sum += v[j];
      if (row < N) store_y(y, (int64_t)c * N + row, sum, ydt);
    }
    PH_MARK(kPhEnd);
    PH_PUT(kPhSlices, 1ull);
    PH_FLUSH(NW);
    return;
  }
  // Each wave's first two units are static (wave, wave + NW); the counter hands out
  // the rest.
  constexpr bool rot = MODE == kRotated || rot1;
  for (int s = s_begin; s < s_end; ++s) {
    const int k0 = s * SPL * 512;
    const int kw = min(K - k0, nsl * 128);  // rotated width of the slice
    const int per_row = rot ? kw / 8 : nsl * 16;  // x chunks per batch row
    // batch row of x chunk t: per_row = 64 SPL without a rotation
    // batch row of the plain layout's chunks tw .. tw + 63 (per_row = 64 SPL)
    auto row_of_wave = [&](int tw) { return fdiv(tw >> 6, SPL, spl_m); };
    // With several slices, an opaque copy of the thread index keeps the compiler from
    // hoisting the staging index math out of the slice loop (it would stay live, in
    // registers the decode needs, for the whole kernel).
    int tid = threadIdx.x, wv = wave;
    if constexpr (MODE != kFlat && !rot1 && !flat1) {
      asm volatile("" : "+v"(tid));
      asm volatile("" : "+s"(wv));
    }
    // kRotDA: the first NWR waves rotate x; the others decode ahead (wave-uniform)
    const bool rw = !da || wave < NWR;
    XPre<XP> xp;
    XRot xr;
    if constexpr (rot) {
      if (rw) rot_preload<NWR>(xr, xrs, K, B, k0, kw, fwht_block, tid);
    } else
      x_preload<NT, XP, flat1>(xp, xrs, K, k0, per_row, B * per_row, row_of_wave, wv, tid);
    // MX: the thread's first scale entry is requested with its x (a slice has at most
    // kLdsLimit / 272 < NT entries whenever its x fits LDS, so this is usually all of them)
    uint2 sc_first = {0u, 0u};
    if constexpr (mx)
      if (tid < B * nsl) sc_first = sc_load(tid, k0);
    if (s == 0) PH_MARK(kPhXIssued);
    if constexpr (MODE != kFlat && !rot1 && !flat1) {
      if (s == nslices - 1 && spl_last != SPL) {  // a last slice with fewer spans
        sp = spl_last;
        sp_m = 0xFFFFFFFFu / (unsigned)spl_last;  // floor(2^32 / sp), or one less: fdiv fixes it
        nu = (t1 - t0) * spl_last;
      }
    }
    int u0 = wave, u1 = wave + NW;
    if constexpr (da) {
      // Static units: decode-ahead wave d = wave - NWR takes unit d and decodes it into
      // registers while the others rotate x; rotating wave r takes NWR + r before its rotation
      // and 2 NWR + r after it.  The counter hands out the rest (a decode-ahead wave takes its
      // second unit from it before the staging barrier, so that unit is in flight across it).
      // The counter, the rotating waves' own barrier counter, the tile counts and the zero
      // block are set before a workgroup barrier, which also queues the decode-ahead waves'
      // weight requests behind the rotation's x.
      if (threadIdx.x == 0) {
        counter[0] = 3 * NWR;
        counter[1] = 0;
      }
      for (int i = threadIdx.x; i < t1 - t0; i += NT) tile_cnt[i] = 0;
      if (threadIdx.x < zero_bytes(FMT) / 16)
        reinterpret_cast<u32x4*>(zeros)[threadIdx.x] = u32x4{0u, 0u, 0u, 0u};
      __syncthreads();
      Dec dec;
      if (rw) {
        u0 = NWR + wave;
        u1 = u0 + NWR;
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): x
        if (s == 0) PH_MARK(kPhXArrived);
        issue(s, u0, ring[0]);
        if (s == 0) PH_MARK(kPhU0Issued);
        stage_fwht<NWR, true, true>(xst, reinterpret_cast<float*>(xst + B * RS), xr, xrs, K, B,
                                    k0, kw, nsl, RS, fwht_block, fwht_scale, tid, counter + 1 PH_ARG);
        if constexpr (da_all) {
          issue(s, u1, ring[1]);
          unit_decode<FMT, XDT>(ring[0], dec);
        }
      } else {
        u0 = wave - NWR;
        issue(s, u0, ring[0]);
        if (s == 0) PH_MARK(kPhU0Issued);
        unit_decode<FMT, XDT>(ring[0], dec);  // waits for its weights, not for x
#ifdef FB_PHASE_TRACE
        // the mark after the decode's last result, not wherever the scheduler would put it
#pragma unroll
        for (int j = 0; j < 16; ++j) asm volatile("" ::"v"(dec.a[j]));
#endif
        if (s == 0) PH_MARK(kPhDecodedAhead);
        u1 = __builtin_amdgcn_readfirstlane(grab());
        issue(s, u1, ring[1]);
      }
      __syncthreads();  // x staged
      PH_MARK(kPhStaged);
      if (rw && !da_all) {
        issue(s, u1, ring[1]);
        __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the compute
        if (u0 < nu) process(ring[0], s, u0);
      } else if (u0 < nu) {
        const int lt = tile_of(u0);
        const int span = u0 - lt * sp;
        finish(unit_mfma<XDT>(dec, xl + span * xspan), s, lt, span);
      }
    } else {
      // the rotation cannot start before its x has arrived, and x loads queued behind the
      // first weight unit arrive later: wait for x first
      if constexpr (rot) __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      if (rot && s == 0) PH_MARK(kPhXArrived);
      // E2M1 at batch >= 2 (K-sliced, or in one slice with at most 4 units per wave), and GF4
      // in one K-slice on 8 waves with at most 4 units per wave: the workgroup's x requests
      // all enter the CU's load queue before any weight request (a wave that starts late
      // would otherwise queue its x behind the others' first units, and the staging barrier
      // waits for it).  With more units per wave in one slice the first unit's delay costs
      // more than x gains.
      if constexpr (!rot && !flat1 && (FMT == FB_FMT_E2M1 || (NW == 8 && MODE == kFlat)))
        if (s == s_begin && ((FMT == FB_FMT_E2M1 && MODE != kFlat) || nu <= 4 * NW))
          __builtin_amdgcn_s_barrier();
      issue(s, u0, ring[0]);
      if (s == 0) PH_MARK(kPhU0Issued);
      // The next slice's x (into registers) and first weight unit are requested before the
      // barrier that closes the previous slice, so their latency overlaps the slowest wave.
      if (s > s_begin) {  // every wave is done with the previous slice: x may be restaged
        __syncthreads();
        if (threadIdx.x == 0) *counter = 2 * NW;
      }
      if (s == s_begin) {
        // a workgroup may own more row tiles than it has threads (a long N over a short K)
        if constexpr (tile_reduce)
          for (int i = threadIdx.x; i < t1 - t0; i += NT) tile_cnt[i] = 0;
        if (threadIdx.x == 0) *counter = 2 * NW;
        if (threadIdx.x < zero_bytes(FMT) / 16)
          reinterpret_cast<u32x4*>(zeros)[threadIdx.x] = u32x4{0u, 0u, 0u, 0u};
      }
      if constexpr (rot)
        stage_fwht<NW>(xst, reinterpret_cast<float*>(xst + B * RS), xr, xrs, K, B, k0, kw, nsl,
                       RS, fwht_block, fwht_scale, tid, nullptr PH_ARG);
      else
        stage_plain<NT, XP, flat1>(xst, xp, xrs, K, B, k0, nsl, RS, row_of_wave, wv, tid);
      if constexpr (mx) {
        if (tid < B * nsl) sc_store(tid, sc_first);
        for (int i = tid + NT; i < B * nsl; i += NT) sc_store(i, sc_load(i, k0));
      }
      __syncthreads();  // x staged, counter set
      PH_MARK(s == 0 ? kPhStaged : s == 1 ? kPhStaged1 : kPhStaged2);
      issue(s, u1, ring[1]);
      __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the compute
      if (u0 < nu) process(ring[0], s, u0);
    }
    if (s == 0) PH_MARK(kPhUnit0);
    int un = grab();
    for (;;) {
      u0 = __builtin_amdgcn_readfirstlane(un);
      un = grab();
      issue(s, u0, ring[0]);
      __builtin_amdgcn_sched_barrier(0);
      if (u1 >= nu) break;
      process(ring[1], s, u1);
      u1 = __builtin_amdgcn_readfirstlane(un);
      un = grab();
      issue(s, u1, ring[1]);
      __builtin_amdgcn_sched_barrier(0);
      if (u0 >= nu) break;
      process(ring[0], s, u0);
    }
    PH_MARK(s == nslices - 1 ? kPhLoopEnd : s == 0 ? kPhSliceEnd0 : kPhSliceEnd1);
  }
  if constexpr (!tile_reduce) {
    __syncthreads();  // every slice done: slots are complete
    PH_MARK(kPhFinalBar);
    // y[col][row] = sum over the spans of the tile, in span order (kSplitK: the spans of
    // this workgroup's part, sp of them)
    const int nt = t1 - t0;
    const int nsp = splitk ? sp : SPL;
    for (int e = threadIdx.x; e < nt * 256; e += NT) {
      const int c = e & 15;
      if (c >= B) continue;
      const int r = (e >> 4) & 15;
      const int lt = e >> 8;
      const int row = (t0 + lt) * 16 + r;
      const f32x4* sl = slots + ((size_t)lt * SPL * 4 + (r >> 2)) * B + c;
      float sum = 0.0f;
      for (int j = 0; j < nsp; ++j) sum += sl[(size_t)j * 4 * B][r & 3];
      if (row < N) store_y(yo, (int64_t)c * N + row, sum, ydt);
    }
  }
  PH_MARK(kPhEnd);
  PH_PUT(kPhSlices, (unsigned long long)nslices);
  PH_FLUSH(NW);
}

// ---------------------------------------------------------------------------------
// The split-K sum: y[i] = ((part_0[i] + part_1[i]) + ...) + part_{P-1}[i], fp32, in part
// order whichever workgroup finished first; four outputs per thread, 16-byte reads where
// the batch-by-rows count allows.  P (4 or 8) is a template argument so that the P reads
// of a thread are issued back to back before the first add waits for them.
template <int P>
__global__ __launch_bounds__(256) void splitk_sum(const float* __restrict__ part, int64_t n,
                                                  void* __restrict__ y, int ydt) {
  const int64_t i0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i0 >= n) return;
  if (i0 + 4 <= n && (n & 3) == 0) {
    f32x4 v[P];
#pragma unroll
    for (int p = 0; p < P; ++p)
      v[p] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(part + (int64_t)p * n + i0));
    f32x4 a = v[0];
#pragma unroll
    for (int p = 1; p < P; ++p) a += v[p];
    if (ydt == FB_DT_F32) {
      *reinterpret_cast<f32x4*>(static_cast<float*>(y) + i0) = a;
    } else {  // two 4-byte stores: y is only known to be 4-byte aligned
      unsigned h[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        h[j] = ydt == FB_DT_F16 ? __builtin_bit_cast(unsigned short, (_Float16)a[j])
                                : __builtin_bit_cast(unsigned short, (__bf16)a[j]);
      unsigned* yo = reinterpret_cast<unsigned*>(static_cast<uint16_t*>(y) + i0);
      yo[0] = h[0] | (h[1] << 16);
      yo[1] = h[2] | (h[3] << 16);
    }
  } else {
    for (int64_t i = i0; i < min(n, i0 + 4); ++i) {
      float a = part[i];
      for (int p = 1; p < P; ++p) a += part[(int64_t)p * n + i];
      store_y(y, i, a, ydt);
    }
  }
}

// Device decode: one thread per item writes 128 values of row n.
// ---------------------------------------------------------------------------------
template <int FMT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ w,
                                                      void* __restrict__ out, int N, int K,
                                                      int odt) {
  constexpr int BB = FMT == FB_FMT_GF4 ? fb::kGf4BlockBytes : fb::kE2m1BlockBytes;
  const int G = K >> 7;
  const int GS = (G + 3) >> 2;
  const int64_t item = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (item >= (int64_t)N * G) return;
  const int n = (int)(item / G);
  const int g = (int)(item - (int64_t)n * G);
  Rec<FMT> r;
  load_rec_global<FMT>(w + ((int64_t)(n >> 4) * GS + (g >> 2)) * BB, (n & 15) + 16 * (g & 3), r);
  const int64_t o0 = (int64_t)n * K + g * 128;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int e = FMT == FB_FMT_GF4 ? 0 : (int)((r.t0.x >> (8 * c)) & 0xFFu) - 127;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      u32x4 pr;
      if constexpr (FMT == FB_FMT_GF4)
        pr = gf4_decode8(r.nib[c][d], r.t0, r.t1);
      else
        pr = e2m1_decode8<FB_DT_BF16>(r.nib[c][d], 1.0f);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const unsigned bits = (pr[jj] >> (16 * h)) & 0xFFFFu;
          float v;
          if constexpr (FMT == FB_FMT_GF4)
            v = (float)__builtin_bit_cast(_Float16, (unsigned short)bits);
          else
            v = __builtin_ldexpf(__builtin_bit_cast(float, bits << 16), e);
          const int64_t o = o0 + c * 32 + d * 8 + jj * 2 + h;
          if (odt == FB_DT_F32) {
            static_cast<float*>(out)[o] = v;
          } else if (odt == FB_DT_F16) {
            if constexpr (FMT == FB_FMT_GF4)
              static_cast<unsigned short*>(out)[o] = (unsigned short)bits;
            else
              static_cast<_Float16*>(out)[o] = (_Float16)v;
          } else {
            static_cast<__bf16*>(out)[o] = (__bf16)v;
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// Rotation of x once per call, for batches where every workgroup rotating all of x in its
// prologue would cost more than a launch: workgroup (c, b) rotates row b's values
// [4096c, 4096c + 4096) with stage_fwht (the same arithmetic as the GEMV's own prologue, so
// the fp16 values are the ones the GEMV would stage) and writes them to xo [B, K].
// ---------------------------------------------------------------------------------
constexpr int kRotPiece = 4096;
constexpr int kRotWaves = 4;

__host__ __device__ inline int rot_lds_bytes(int kw) {
  return ((x_row_stride(kw / 128) + 15) & ~15) + fpad(kw) * 4 + 64;
}

template <int NW>
__global__ __launch_bounds__(NW * 64) void rotate_kernel(const uint16_t* __restrict__ x,
                                                         uint16_t* __restrict__ xo, int K,
                                                         int fb, float sc) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int c = blockIdx.x, b = blockIdx.y;
  const int k0 = c * kRotPiece;
  const int kw = min(kRotPiece, K - k0);  // a multiple of fb and of 128
  const int nsl = kw / 128;
  const int RS = x_row_stride(nsl);
  float* F = reinterpret_cast<float*>(lds + ((RS + 15) & ~15));
  const int tid = threadIdx.x;
  const uint16_t* xrow = x + (int64_t)b * K;
  const rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(xrow), (short)0,
                                                       K * 2, kRsrcWord3);
  XRot xr;
  PH_DECL  // not written out: the trace covers the GEMV
  rot_preload<NW>(xr, xrs, K, 1, k0, kw, fb, tid);
  stage_fwht<NW>(lds, F, xr, xrs, K, 1, k0, kw, nsl, RS, fb, sc, tid, nullptr PH_ARG);
  __syncthreads();
  uint16_t* orow = xo + (int64_t)b * K + k0;
  for (int t = tid; t < kw / 8; t += NW * 64) {
    const int g = t >> 4, e = (t & 15) * 8;
    *reinterpret_cast<u32x4*>(orow + g * 128 + e) =
        *reinterpret_cast<const u32x4*>(lds + g * kSliceBytes + e * 2);
  }
}

// ---------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------
constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];

int cu_count(int dev) {
  if (dev < 0 || dev >= kMaxDevices) return 256;
  int v = g_cu_count[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  g_cu_count[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

struct Plan {
  int S = 0;     // K-slices staged one after the other
  int SPL = 0;   // spans per slice (the last slice: GS - (S - 1) * SPL)
  int grid = 0;  // workgroups
  int GS = 0;    // spans per row
  int tq = 0;    // row tiles per workgroup (the first tr workgroups take one more)
  int tr = 0;
  int nw = 0;    // waves per workgroup: 16 (one workgroup per CU) or 8 (two per CU)
  int xp = 4;    // x chunks each thread preloads per slice: 4, or 8 for larger slices
  size_t lds = 0;
  int P = 0;     // kSplitK: K-parts run side by side (grid grid x P); 0: slices in turn
  bool da = false;      // kRotDA: batch-1 rotation with decode-ahead waves
  bool da_all = false;  // kRotDAall: the same, every wave decoding ahead (one unit per wave)
  bool spanx = false;   // kSpanX: each wave stages the x of its own spans
};



// The rotation's normalisation 1 / sqrt(b), rounded as fp32 (correctly rounded sqrt and
// division, so the same value the device would compute).
float fwht_scale(int fb) { return fb ? 1.0f / std::sqrt((float)fb) : 1.0f; }

// Multiplier of fdiv: floor(2^32 / d), or 2^32 - 1 for d = 1.
unsigned div_magic(int d) { return d == 1 ? 0xFFFFFFFFu : (unsigned)((1ull << 32) / (unsigned)d); }

// LDS of one workgroup: the unit counter, the zero block that MFMA columns past the batch
// read, staged x, and one partial-sum slot per unit.
size_t plan_lds(const fb_shape_t* s, int tpw, int SPL) {
  // batch 1 adds the per-tile unit counts of the tile-by-tile reduction
  return (size_t)x_lds_bytes(s->B, s->K, SPL, s->fwht_block) + (size_t)tpw * SPL * 64 * s->B +
         (s->B == 1 ? (size_t)((tpw * 4 + 15) & ~15) : 0) + 16 + zero_bytes(s->fmt);
}

// The fewest K-slices whose LDS fits.
// - Batch-1 GF4 / E2M1 layers whose x fits one slice, rotated or not: one 8-wave workgroup
//   per CU (up to the number of row tiles), run by the max-ILP copy of the kernel, which holds
//   183 VGPRs (GF4, unrotated) so that only one such workgroup fits a CU.  Measured against 16 waves with
//   the default scheduling, same box, median us: GF4 8192 -> 28672 29.79 -> 28.93,
//   28672 -> 8192 30.16 -> 29.31, 4096 -> 28672 17.47 -> 16.55, 4096 -> 14336 10.80 -> 9.96,
//   4096 -> 11008 8.77 -> 8.19; E2M1 8192 -> 28672 20.58 -> 20.28; the rest within 0.1.
//   Rotated, against 16 waves on the rotated kernel's max-ILP copy: 4096^2 7.27 -> 6.96,
//   4096 -> 11008 10.58 -> 10.06, 11008 -> 4096 10.35 -> 9.60, 8192^2 14.45 -> 13.95.
// - Unrotated GF4 (and E2M1, exact or on the native FP4 path) at batch 2-16 with at most 2
//   row tiles per CU (GF4: or at most 64 units per workgroup), whose x fits one K-slice, or
//   two of at most 2 units per wave each: the same (one 8-wave
//   workgroup per CU on the max-ILP copy, x preloaded 16 chunks per thread where it needs
//   them).  Measured against 16 waves, same box, median us (bitwise-equal outputs):
//   - GF4, one slice: 8192^2 B=2 12.71 -> 11.61, B=4 12.92 -> 11.85, B=8 13.63 -> 12.87;
//     4096^2 B=2 6.06 -> 5.36, B=4 6.23 -> 5.62, B=8 6.35 -> 5.85; 28672 -> 8192 B=2
//     31.09 -> 30.64;
//   - GF4, two slices: 11008 -> 4096 B=8 12.31 -> 11.60, 8192^2 B=16 15.49 -> 15.18,
//     4096^2 B=16 7.12 -> 6.73; but 28672 -> 8192 B=4 (7 units per wave per slice) 33.24 on
//     16 waves against 33.60, and with four slices (28672 -> 8192 B=8) 39.10 / 41.31;
//   - E2M1 (bf16 x), another box: 8192^2 B=8 9.04 -> 8.75, B=16 11.92 -> 11.67, 4096^2 B=4
//     4.89 -> 4.32, 11008 -> 4096 B=8 9.48 -> 9.14 (an earlier build's 8-wave E2M1, with x
//     past an 8-chunk preload loaded behind the first unit, had been slower: 8192^2 B=8
//     8.90 / 9.48); with fp16 x: 8192^2 B=2 8.44 -> 7.96, B=8 8.89 -> 8.71, B=16 11.84 ->
//     11.66, 4096^2 B=4 4.81 -> 4.33;
//   - the native FP4 path (fb_gemv_mx, split included), another box: 8192^2 B=16 14.79 ->
//     13.99, 11008 -> 4096 B=8 12.30 -> 11.61, 4096^2 B=4 6.81 -> 6.26, B=8 7.33 -> 7.19;
//     8192^2 B=2 9.82 -> 9.76, B=4 10.13 -> 10.20, B=8 10.96 -> 11.17;
//   - GF4 on 3-7 row tiles per CU of short rows (at most 64 units per workgroup):
//     4096 -> 11008 B=4 10.31 -> 8.79, B=8 10.43 -> 9.20, B=16 12.13 -> 11.53; 4096 -> 28672
//     B=2 18.07 -> 17.36, B=4 18.23 -> 17.40; 8192 -> 16384 B=4 20.43 -> 19.91; 8192 ->
//     14336 B=2 18.33 -> 18.02; but two slices of more than 2 units per wave were slower
//     (4096 -> 28672 B=16 21.99 / 22.62, 8192 -> 14336 B=8 20.75 / 21.17), and so was E2M1
//     there (4096 -> 28672 B=8 12.39 / 12.67);
//   - with more units per workgroup 16 waves were faster (GF4 8192 -> 28672, 112 units:
//     B=2 30.53 / 30.68, B=4 30.71 / 31.39).
// - The native FP4 path's batch-1 layers with few row tiles per CU (at most 2) and LDS that
//   fits twice in a CU: two 8-wave workgroups per CU.
// - Otherwise one 16-wave workgroup per CU (batches of more row tiles per CU, larger x, E2M1
//   with fp16 x, rotated batches).
bool make_plan_staged(const fb_shape_t* s, int cus, Plan& pl) {
  const int GS = (s->K / 128 + 3) / 4;
  const int T = (s->N + 15) / 16;
  const bool one8 = (s->B == 1 && s->fmt != kFmtMx) ||
                    ((s->fmt == FB_FMT_GF4 && s->x_dtype == FB_DT_F16) ||
                     s->fmt == FB_FMT_E2M1 ||
                     (s->fmt == kFmtMx && s->B >= 2)) &&
                     !s->fwht_block && s->B <= 16 &&
                     (T <= 2 * cus || (s->fmt == FB_FMT_GF4 && (T + cus - 1) / cus * GS <= 64));
  const bool half = one8 || (!s->fwht_block && s->B == 1 && T <= 2 * cus);
  for (int pass = half ? 0 : 1; pass < 2; ++pass) {
    const int nw = pass == 0 ? kWaves / 2 : kWaves;
    const size_t limit = pass == 0 && !one8 ? (size_t)kLdsLimit / 2 : (size_t)kLdsLimit;
    const int grid = std::max(1, std::min(T, pass == 0 && !one8 ? 2 * cus : cus));
    const int tpw = (T + grid - 1) / grid;  // most tiles a workgroup owns
    for (int S = 1; S <= GS; ++S) {
      int SPL = (GS + S - 1) / S;  // spans per slice; the last slice may have fewer
      if (S > 1 && s->fwht_block > 512) {  // a slice holds whole rotation blocks
        const int bs = s->fwht_block / 512;
        SPL = (SPL + bs - 1) / bs * bs;
      }
      if ((S - 1) * SPL >= GS) continue;  // the last slice would have no span
      // 8-wave workgroups with one K-slice at batch 1, at most two at batch 2-16
      if (pass == 0 && S > (s->B == 1 ? 1 : 2)) break;
      // two slices only where each wave has few units per slice
      if (pass == 0 && S == 2 && tpw * SPL > 2 * nw) break;
      const size_t lds = plan_lds(s, tpw, SPL);
      if (lds > limit) continue;
      pl.S = S;
      pl.SPL = SPL;
      pl.grid = grid;
      pl.GS = GS;
      pl.tq = T / grid;
      pl.tr = T % grid;
      pl.nw = nw;
      // 16-byte x chunks per thread: 4 or 8 (16 only in the 8-wave batch 2-16 plan)
      const int chunks = (s->B * SPL + nw - 1) / nw;
      pl.xp = chunks <= 4 ? 4 : chunks <= 8 || nw == kWaves || s->B == 1 ? 8 : 16;
      pl.lds = lds;
      // The 8-wave rotated plan with decode-ahead waves (kRotDA) where half the waves can
      // rotate x: blocks larger than one 256-value sub-block (whose rotation has a barrier's
      // wait for the other waves to fill) and x within the rotating waves' preloads.
      // Measured against kRot1, same box, median us: GF4 4096^2 b=4096 6.92 -> 6.23, 4096 ->
      // 11008 10.07 -> 9.57 (outputs bitwise equal).  Two units decoded ahead per wave: 6.27,
      // 10.43 (the staging barrier waited for the second); 16-wave workgroups (8 rotating, 8
      // decoding ahead, 128 registers): 6.67, 10.36.
      pl.da = s->fwht_block > 256 && s->B == 1 && S == 1 && pass == 0 &&
              (s->K + 255) / 256 <= kWaves / 4 * kXPre;
      // every wave decoding ahead where a workgroup owns at most one unit per wave; measured
      // on 4096^2 (one tile of 8 units per workgroup) 5.66 -> 5.46 us, and slower where the
      // workgroups own more (4096 -> 11008: 9.37 -> 9.93)
      pl.da_all = pl.da && (pl.tq + (pl.tr ? 1 : 0)) * SPL <= nw;
      return true;
    }
  }
  return false;
}

// kSpanX (batch >= 2, unrotated): each of 8 waves stages the x of its own spans, one span
// (B x 512 values) at a time, in an LDS region of its own, instead of the workgroup staging
// x K-slice by K-slice behind barriers; the wave adds its units' sums per row tile in
// registers (at most 8 tiles).  Taken where the staged plan needs two or more K-slices, each
// wave owns at least two units (GF4: at least two spans), and the workgroup at most 4 row
// tiles (8 at batch 8-16); over split-K where a wave owns 4 or more spans and the row tiles
// fill every CU (split-K's parts multiply the workgroups of fewer tiles).  Measured against
// the plans before it on 46 shapes, same box, median us of 9 regions (outputs within fp16
// rounding of them: another order of the same fp32 sums):
// - 8192^2 B=12: GF4 16.12 -> 14.26, E2M1 10.94 -> 9.76; B=16: GF4 16.17 -> 15.33, E2M1
//   11.71 -> 10.46 (another box 14.86 -> 14.10, 11.65 -> 10.25);
// - 8192 -> 28672 B=16: GF4 39.36 -> 35.81, E2M1 25.80 -> 24.62 (another box 34.80 -> 34.39,
//   24.23 / 24.32);
// - 28672 -> 8192: B=3 E2M1 22.70 -> 20.94 (GF4 33.24 / 33.46), B=8 GF4 38.37 -> 36.23,
//   E2M1 25.55 -> 23.49, B=16 GF4 43.77 -> 40.62, E2M1 35.37 -> 29.13 (over split-K);
// - 16384 -> 4096 B=16: GF4 20.69 -> 17.54, E2M1 16.89 -> 13.12 (over split-K; at B=12
//   16.26 / 16.49 and 11.38 / 11.83); 8192 -> 16384 B=16: GF4 26.55 -> 23.38, E2M1 18.81 ->
//   16.01; 11008 -> 4096 B=12: GF4 13.58 -> 12.45, E2M1 10.57 -> 9.36; E2M1 4096 -> 11008
//   B=16 9.63 -> 8.49;
// - GF4 with one span per wave was mixed (4096 -> 11008 B=16 12.05 / 12.75 and 11.53 /
//   10.76, 4096 -> 28672 B=16 23.55 / 24.08), so GF4 takes it from two spans per wave; the
//   one-slice plans stay (8192^2 B=8: GF4 11.76 / 12.71, E2M1 8.70 / 8.98), and so does
//   split-K over fewer spans per wave (11008 -> 4096 B=16: GF4 11.85 / 12.67, E2M1 9.92 /
//   10.19);
// - 7 row tiles at batch 8-12, measured after the epilogue's slot reads were batched (they
//   are the same sums in the same order as the two staged K-slices there, so the bits are
//   equal): 8192 -> 28672 B=8 GF4 32.80 -> 32.54, E2M1 22.41 / 22.47; B=12 GF4 34.40 ->
//   33.74, E2M1 23.36 -> 23.10;
// - the native FP4 path (fb_gemv_mx, split per call), same box: 8192^2 B=16 13.92 -> 13.16,
//   4096 -> 11008 B=16 11.85 -> 9.97, 28672 -> 8192 B=8 28.50 -> 27.53, 11008 -> 4096 B=8
//   11.63 -> 11.19, 8192 -> 28672 B=16 26.48 -> 26.32; but 7 row tiles at batch 8 slower
//   (8192 -> 28672 B=8 23.75 / 24.72), so there it takes 8 row tiles at batch 16 only.
bool spanx_plan(const fb_shape_t* s, int cus, const Plan& staged, Plan& pl) {
  if (s->B < 2 || s->B > 16 || s->fwht_block || staged.S < 2) return false;
  const int GS = (s->K / 128 + 3) / 4;
  const int T = (s->N + 15) / 16;
  const int grid = std::max(1, std::min(T, cus));
  const int tpw = (T + grid - 1) / grid;
  const int nw = kWaves / 2;
  // at most 4 row tiles per workgroup; 8 at batch 8-16 (the native FP4 path: at batch 16)
  const int tmax = s->B == 16 || (s->B >= 8 && s->fmt != kFmtMx) ? 8 : 4;
  if (tpw > tmax || tpw * ((GS + nw - 1) / nw) < 2) return false;
  if (s->fmt == FB_FMT_GF4 && GS <= nw) return false;  // one span per wave
  // the waves' x regions, which the (tile, wave) slots take over after the last unit
  const size_t lds = 16 + zero_bytes(s->fmt) +
                     std::max((size_t)nw * s->B * x_row_stride(4), (size_t)tpw * nw * s->B * 64) +
                     nw * 4;  // the waves' unit counts
  if (lds > (size_t)kLdsLimit) return false;
  pl = Plan();
  pl.S = 1;
  pl.SPL = GS;
  pl.grid = grid;
  pl.GS = GS;
  pl.tq = T / grid;
  pl.tr = T % grid;
  pl.nw = nw;
  pl.xp = tpw <= 2 ? 2 : tpw <= 4 ? 4 : 8;  // the kernel's register count of row tiles
  pl.lds = lds;
  pl.spanx = true;
  return true;
}

bool make_plan(const fb_shape_t* s, int cus, Plan& pl) {
  if (!make_plan_staged(s, cus, pl)) return false;
  Plan sx;
  if (spanx_plan(s, cus, pl, sx)) pl = sx;
  return true;
}

// kSplitK (batch >= 2, unrotated): the K-slices of the sliced layout run side by side, P
// workgroups per row range, each staging only its own part of x, with no slice barrier.  The
// parts' fp32 sums (P * B * N * 4 bytes) go to the caller's workspace and splitk_sum adds
// them in part order (one more launch, and the sums' traffic).  Measured on MI355X against
// the slices in turn, it pays only where the sliced plan needs 3 or more slices of a long K
// (K >= 10240) with at most 2 row tiles per workgroup: 11008 -> 4096 at batch 16, GF4
// 16.7 -> 14.3 us and E2M1 13.4 -> 11.1 us (P = 4).  With 2 slices it was within +-1 us
// either way (batch 8 at K = 11008, batch 4 at K = 28672), and on layers of more row tiles
// per workgroup (8192 -> 8192, 8192 -> 28672 at batch 8/16) up to 8 us slower.  P: the
// sliced plan's slice count rounded up to a power of two (at most 8), if its LDS fits.
// 0 where it does not apply.
#if defined(FB_PHASE_TRACE) && !defined(FB_GEMV_ILP_TU)
// Diagnostic library only: a part count that overrides the choice below (fb_phase_force_parts;
// 0 = the library's own choice, -1 = never, 2 / 4 / 8 = that many parts for every unrotated
// batch >= 2 whose plan fits).
std::atomic<int> g_force_parts{0};
int forced_parts() { return g_force_parts.load(std::memory_order_relaxed); }
#else
constexpr int forced_parts() { return 0; }
#endif

int splitk_parts(const fb_shape_t* s, int cus, Plan* out) {
  const int forced = forced_parts();
  if (forced < 0 || s->fwht_block || s->B < 2) return 0;
  const int GS = (s->K / 128 + 3) / 4;
  const int T = (s->N + 15) / 16;
  int P = forced;
  if (!P) {
    if (s->K < 10240) return 0;
    Plan std_pl, sx;
    if (!make_plan_staged(s, cus, std_pl) || std_pl.S < 3) return 0;
    if ((T + std_pl.grid - 1) / std_pl.grid > 2) return 0;
    if (GS >= 32 && T >= cus && spanx_plan(s, cus, std_pl, sx)) return 0;  // kSpanX is faster
    P = 2;
    while (P < std_pl.S) P *= 2;
  }
  if (P > 8 || P > GS) return 0;
  const int SPL = (GS + P - 1) / P;
  if ((P - 1) * SPL >= GS) return 0;  // the last part would have no span
  const int gx = std::max(1, std::min(T, cus / P));
  const size_t lds = plan_lds(s, (T + gx - 1) / gx, SPL);
  if (lds > (size_t)kLdsLimit) return 0;
  if (out) {
    out->S = P;
    out->SPL = SPL;
    out->grid = gx;
    out->GS = GS;
    out->tq = T / gx;
    out->tr = T % gx;
    // 8-wave workgroups on the max-ILP copy (each owns a few row tiles of one part); measured
    // against 16 waves, same box, median us: E2M1 11008 -> 4096 B=16 10.27 -> 9.94 and 10.32
    // -> 10.06, with fp16 x 10.28 -> 9.88; GF4 13.89 / 13.84, 13.80 / 13.78 (bitwise equal)
    out->nw = s->fmt == kFmtMx ? kWaves : kWaves / 2;
    const int chunks = (s->B * SPL + out->nw - 1) / out->nw;
    out->xp = chunks <= 4 ? 4 : chunks <= 8 ? 8 : 16;
    out->lds = lds;
    out->P = P;
  }
  return P;
}

size_t splitk_bytes(const fb_shape_t* s, int P) {
  return P ? ((size_t)P * s->B * s->N * 4 + 255) & ~size_t(255) : 0;
}

int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  return cu_count(dev);
}

template <int FMT, int XDT, int MODE, int NW, int XP>
int launch_gemv(const void* wdev, const void* x, void* y, const fb_shape_t* s, const Plan& pl,
                hipStream_t stream) {
  auto kern = gemv_kernel<FMT, XDT, MODE, NW, XP>;
  // the LDS limit is a per-device attribute of the kernel: set once on each device
  static std::atomic<uint64_t> attr_set{0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return FB_ERR_HIP;
  const uint64_t bit = dev >= 0 && dev < 64 ? uint64_t{1} << dev : 0;
  if (!bit || !(attr_set.load(std::memory_order_acquire) & bit)) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kLdsLimit) != hipSuccess)
      return FB_ERR_HIP;
    attr_set.fetch_or(bit, std::memory_order_release);
  }
  hipLaunchKernelGGL(kern, dim3(pl.grid, pl.P ? pl.P : 1), dim3(NW * 64), pl.lds, stream,
                     static_cast<const uint8_t*>(wdev), x, s->K, s->B, pl.SPL, pl.GS, pl.tq,
                     pl.tr, div_magic(pl.SPL), pl.S, s->fwht_block,
                     x_row_stride(MODE == kSpanX ? 4 : pl.SPL * 4),
                     fwht_scale(s->fwht_block), y, s->N, s->y_dtype
                     PH_KARG((size_t)pl.grid * (pl.P ? pl.P : 1) * NW * 64));
  return hipGetLastError() == hipSuccess ? FB_OK : FB_ERR_HIP;
}

// The host side from here to the end of the file is compiled in the default unit only, so
// that the max-ILP unit instantiates no kernel but its own.
#ifndef FB_GEMV_ILP_TU

template <int FMT, int XDT>
int launch_mode(int mode, const void* wdev, const void* x, void* y, const fb_shape_t* s,
                const Plan& pl, hipStream_t stream) {
  const bool deep = pl.xp >= 8;
  // fb_ilp::launch starts these kernels (instantiated in the max-ILP unit, not here)
  constexpr bool ilp = FMT != kFmtMx;
  // the native FP4 path's 8-wave batch 2-16 plan (its batch-1 layers, two 8-wave workgroups
  // per CU, run below in this unit)
  if constexpr (FMT == kFmtMx)
    if (((mode == kFlat || mode == kSliced) && pl.nw == kWaves / 2) || mode == kSpanX)
      return fb_ilp::launch(FMT, XDT, mode, wdev, x, y, s, pl.grid, pl.SPL, pl.GS, pl.tq, pl.tr,
                            pl.S, pl.lds, pl.xp, stream);
  // the max-ILP copies: the rotated batch-1 kernel, the 8-wave batch-1 one and the 8-wave
  // batch 2-16 ones of GF4, E2M1 and the native FP4 path (one workgroup per CU: the GF4
  // copies' registers leave room for no second)
  if constexpr (ilp) {
    if ((mode == kRot1 || mode == kFlat1 ||
         mode == kFlat || mode == kSliced) &&
        pl.nw == kWaves / 2)
      return fb_ilp::launch(FMT, XDT,
                            mode != kRot1 ? mode : pl.da_all ? kRotDAall : pl.da ? kRotDA : mode,
                            wdev, x, y, s, pl.grid, pl.SPL, pl.GS, pl.tq, pl.tr, pl.S, pl.lds,
                            pl.xp, stream);
  }
  if constexpr (ilp)
    if (mode == kSpanX)
      return fb_ilp::launch(FMT, XDT, kSpanX, wdev, x, y, s, pl.grid, pl.SPL, pl.GS, pl.tq, pl.tr,
                            pl.S, pl.lds, pl.xp, stream);
  if constexpr (ilp)
    if (mode == kSplitK && pl.nw == kWaves / 2)
      return fb_ilp::launch(FMT, XDT, kSplitK, wdev, x, y, s, pl.grid, pl.SPL, pl.GS, pl.tq, pl.tr,
                            pl.S, pl.lds, pl.xp, stream);
  if (mode == kSplitK)
    return deep ? launch_gemv<FMT, XDT, kSplitK, kWaves, 8>(wdev, x, y, s, pl, stream)
                : launch_gemv<FMT, XDT, kSplitK, kWaves, 4>(wdev, x, y, s, pl, stream);
  if (mode == kFlat1) {
    if (pl.nw == kWaves / 2) {
      if constexpr (!ilp)
        return deep ? launch_gemv<FMT, XDT, kFlat1, kWaves / 2, 8>(wdev, x, y, s, pl, stream)
                    : launch_gemv<FMT, XDT, kFlat1, kWaves / 2, 4>(wdev, x, y, s, pl, stream);
      return FB_ERR_HIP;  // not reached: started by fb_ilp::launch above
    }
    return deep ? launch_gemv<FMT, XDT, kFlat1, kWaves, 8>(wdev, x, y, s, pl, stream)
                : launch_gemv<FMT, XDT, kFlat1, kWaves, 4>(wdev, x, y, s, pl, stream);
  }
  if (mode == kFlat) {
    if (pl.nw == kWaves / 2)
      return deep ? launch_gemv<FMT, XDT, kFlat, kWaves / 2, 8>(wdev, x, y, s, pl, stream)
                  : launch_gemv<FMT, XDT, kFlat, kWaves / 2, 4>(wdev, x, y, s, pl, stream);
    return deep ? launch_gemv<FMT, XDT, kFlat, kWaves, 8>(wdev, x, y, s, pl, stream)
                : launch_gemv<FMT, XDT, kFlat, kWaves, 4>(wdev, x, y, s, pl, stream);
  }
  if (mode == kSliced)
    return deep ? launch_gemv<FMT, XDT, kSliced, kWaves, 8>(wdev, x, y, s, pl, stream)
                : launch_gemv<FMT, XDT, kSliced, kWaves, 4>(wdev, x, y, s, pl, stream);
  if constexpr (FMT == kFmtMx) {
    return FB_ERR_FWHT;  // the split is of unrotated x
  } else {
    // the rotation preloads kXPre 256-value sub-blocks per wave instead
    if (mode == kRot1) {  // 16 waves: a plan that would not fit 8-wave staging (not met)
      if (pl.nw == kWaves) return launch_gemv<FMT, XDT, kRot1, kWaves, 4>(wdev, x, y, s, pl, stream);
      if constexpr (!ilp)
        return launch_gemv<FMT, XDT, kRot1, kWaves / 2, 4>(wdev, x, y, s, pl, stream);
      return FB_ERR_HIP;  // not reached: started by fb_ilp::launch above
    }
    return launch_gemv<FMT, XDT, kRotated, kWaves, 4>(wdev, x, y, s, pl, stream);
  }
}

int launch_plan(const void* wdev, const void* x, void* y, const fb_shape_t* s, const Plan& pl,
                hipStream_t hs) {
  const int mode = s->fwht_block ? (s->B == 1 && pl.S == 1 ? kRot1 : kRotated)
                   : pl.spanx     ? kSpanX
                   : pl.P         ? kSplitK
                   : pl.S > 1     ? kSliced
                   : s->B == 1    ? kFlat1
                                  : kFlat;
  if (s->fmt == FB_FMT_GF4) return launch_mode<FB_FMT_GF4, FB_DT_F16>(mode, wdev, x, y, s, pl, hs);
  if (s->fmt == kFmtMx) return launch_mode<kFmtMx, FB_DT_BF16>(mode, wdev, x, y, s, pl, hs);
  if (s->x_dtype == FB_DT_BF16)
    return launch_mode<FB_FMT_E2M1, FB_DT_BF16>(mode, wdev, x, y, s, pl, hs);
  return launch_mode<FB_FMT_E2M1, FB_DT_F16>(mode, wdev, x, y, s, pl, hs);
}

// Rotated calls with at least this many activation values (B * K) rotate x once
// (rotate_kernel, into the workspace) instead of in the prologue of every workgroup, which
// redoes the whole batch's rotation on every CU.  Measured on MI355X (median us, in-kernel
// against once): 4096x4096 b=4096 B=3 10.8 / 11.6, B=4 12.3 / 11.6, B=16 42.5 / 12.9;
// K=11008 b=256 B=1 11.4 / 12.5, B=2 14.5 / 14.0, B=16 54.3 / 21.0; 8192->28672 b=4096 B=1
// 32.7 / 36.4, B=4 44.9 / 35.8, B=16 176.6 / 43.5.
constexpr int64_t kRotOnceValues = 16384;

size_t rot_once_bytes(const fb_shape_t* s) {
  if (!s->fwht_block || (int64_t)s->B * s->K < kRotOnceValues) return 0;
  return ((size_t)s->B * s->K * 2 + 255) & ~size_t(255);
}

int launch_rotate(const void* x, void* xo, const fb_shape_t* s, hipStream_t hs) {
  const int pieces = (s->K + kRotPiece - 1) / kRotPiece;
  hipLaunchKernelGGL(rotate_kernel<kRotWaves>, dim3(pieces, s->B), dim3(kRotWaves * 64),
                     rot_lds_bytes(std::min(s->K, kRotPiece)), hs,
                     static_cast<const uint16_t*>(x), static_cast<uint16_t*>(xo), s->K,
                     s->fwht_block, fwht_scale(s->fwht_block));
  return hipGetLastError() == hipSuccess ? FB_OK : FB_ERR_HIP;
}

// The GEMV of a validated shape: one launch when a plan fits LDS, else row chunks.
int gemv_planned(const void* wdev, const void* x, void* y, const fb_shape_t* s, int cus,
                 hipStream_t hs, void* ws, size_t ws_bytes) {
  Plan pl;
  // batch 8-16 on layers of few row tiles: the K-parts side by side, through the workspace
  if (ws && splitk_parts(s, cus, &pl) && ws_bytes >= splitk_bytes(s, pl.P)) {
    fb_shape_t sp = *s;
    sp.y_dtype = FB_DT_F32;  // the parts' sums
    const int st = launch_plan(wdev, x, ws, &sp, pl, hs);
    if (st != FB_OK) return st;
    const int64_t n = (int64_t)s->B * s->N;
    const dim3 grid((unsigned)((n + 1023) / 1024));
    const float* part = static_cast<const float*>(ws);
    // P is 4 or 8: splitk_parts takes the sliced plan's slice count (3 or more) rounded up
    // to a power of two, at most 8 (2 only when the diagnostic library forces it)
    if (pl.P == 4)
      hipLaunchKernelGGL(splitk_sum<4>, grid, dim3(256), 0, hs, part, n, y, s->y_dtype);
    else if (pl.P == 8)
      hipLaunchKernelGGL(splitk_sum<8>, grid, dim3(256), 0, hs, part, n, y, s->y_dtype);
    else
      hipLaunchKernelGGL(splitk_sum<2>, grid, dim3(256), 0, hs, part, n, y, s->y_dtype);
    return hipGetLastError() == hipSuccess ? FB_OK : FB_ERR_HIP;
  }
  if (make_plan(s, cus, pl)) return launch_plan(wdev, x, y, s, pl, hs);
  // (an unrotated batch always has a plan: one span per slice fits LDS; the MX kernels find
  // their scales after the whole split, which row chunks would not keep)
  if (s->fmt == kFmtMx) return FB_ERR_LDS;
  // No plan holds the whole batch in LDS (a 4096-wide rotation keeps an fp32 copy of every
  // batch row): the rows run in the largest chunks that fit, each streaming the weights.
  fb_shape_t sc = *s;
  int bc = s->B - 1;
  for (; bc >= 1; --bc) {
    sc.B = bc;
    if (make_plan(&sc, cus, pl)) break;
  }
  if (bc < 1) return FB_ERR_LDS;
  const size_t ysize = s->y_dtype == FB_DT_F32 ? 4 : 2;
  for (int b0 = 0; b0 < s->B; b0 += bc) {
    sc.B = std::min(bc, s->B - b0);
    if (!make_plan(&sc, cus, pl)) return FB_ERR_LDS;
    const int st = launch_plan(wdev, static_cast<const uint8_t*>(x) + (size_t)b0 * s->K * 2,
                               static_cast<uint8_t*>(y) + (size_t)b0 * s->N * ysize, &sc, pl, hs);
    if (st != FB_OK) return st;
  }
  return FB_OK;
}

// fb_gemv behind the ABI.  ws (ws_bytes) holds the once-per-call rotation of larger batches
// (rotated x, first) and the split-K parts' sums (after it); without enough of it the
// rotation runs in every workgroup's prologue and the K-slices in turn.
int gemv_impl(const void* wdev, const void* x, void* y, const fb_shape_t* s, void* ws,
              size_t ws_bytes, hipStream_t hs) {
  if (!s || !wdev || !x || !y) return FB_ERR_NULL;
  int st = fb_validate(s);
  if (st != FB_OK) return st;
  if (s->B > 16) return FB_ERR_BATCH;
  if (!aligned16(wdev) || !aligned16(x) || (reinterpret_cast<uintptr_t>(y) & 3u))
    return FB_ERR_ALIGN;
  if (s->fwht_block && s->x_dtype != FB_DT_F16) return FB_ERR_DTYPE;
  const int cus = device_cus();
  {
    // The kernel addresses a workgroup's blocks with 32-bit offsets from its first block,
    // so the row tiles one workgroup owns (at most ceil(T / min(T, CUs))) must span less
    // than 2^31 bytes.  Under fb_validate's limit of 2^31 groups (192 GiB of GF4 stream)
    // this holds on every device with 128 CUs or more.
    const int64_t T = (s->N + 15) / 16, GS = (s->K / 128 + 3) / 4;
    const int64_t grid = std::min<int64_t>(T, cus);
    if ((T + grid - 1) / grid * GS * fb::block_bytes(s->fmt) > INT32_MAX) return FB_ERR_SHAPE;
  }
  if (ws && (reinterpret_cast<uintptr_t>(ws) & 255u)) ws = nullptr;  // misaligned: unused
  if (!ws) ws_bytes = 0;
  const size_t need = rot_once_bytes(s);
  if (need && ws_bytes >= need) {
    st = launch_rotate(x, ws, s, hs);
    if (st != FB_OK) return st;
    fb_shape_t u = *s;
    u.fwht_block = 0;  // x' is rotated
    return gemv_planned(wdev, ws, y, &u, cus, hs, static_cast<uint8_t*>(ws) + need,
                        ws_bytes - need);
  }
  return gemv_planned(wdev, x, y, s, cus, hs, ws, ws_bytes);
}

// Checks of the native FP4 path's shape: E2M1 weights, bf16 x (8 significant bits, which the
// two E4M3 terms hold), no rotation.
int mx_check(const fb_shape_t* s) {
  const int st = fb_validate(s);
  if (st != FB_OK) return st;
  if (s->fmt != FB_FMT_E2M1) return FB_ERR_FORMAT;
  if (s->x_dtype != FB_DT_BF16) return FB_ERR_DTYPE;
  if (s->fwht_block) return FB_ERR_FWHT;
  if (s->B > 16) return FB_ERR_BATCH;
  return FB_OK;
}

int launch_mx_split(const void* x, void* out, const fb_shape_t* s, hipStream_t hs) {
  const int n8 = s->B * (s->K / 8);  // B K < 2^31 (fb_validate)
  hipLaunchKernelGGL(mx_split_kernel, dim3((n8 + 63) / 64), dim3(64), 0, hs,
                     static_cast<const uint16_t*>(x), static_cast<uint8_t*>(out), n8,
                     mx_scale_offset(s->B, s->K));
  return hipGetLastError() == hipSuccess ? FB_OK : FB_ERR_HIP;
}

// Checks shared by the native FP4 entry points: shape, then the 32-bit block offsets from
// each workgroup's first block (as in gemv_impl).
int mx_gemv_check(const fb_shape_t* s, int cus) {
  const int st = mx_check(s);
  if (st != FB_OK) return st;
  const int64_t T = (s->N + 15) / 16, GS = (s->K / 128 + 3) / 4;
  const int64_t grid = std::min<int64_t>(T, cus);
  if ((T + grid - 1) / grid * GS * fb::kE2m1BlockBytes > INT32_MAX) return FB_ERR_SHAPE;
  return FB_OK;
}

// The GEMV on a split of x (fb_mx_split's layout at xs); ws / ws_bytes may hold the split-K
// parts' sums (without them the K-slices run in turn).
int gemv_mx_split_run(const void* wdev, const void* xs, void* y, const fb_shape_t* s, int cus,
                      void* ws, size_t ws_bytes, hipStream_t hs) {
  fb_shape_t u = *s;
  u.fmt = kFmtMx;
  return gemv_planned(wdev, xs, y, &u, cus, hs, ws, ws_bytes);
}

// fb_gemv_mx behind the ABI: the split into the workspace's head, then the GEMV on it (with
// the split-K parts' sums after the split where the plan runs them side by side).
int gemv_mx_impl(const void* wdev, const void* x, void* y, const fb_shape_t* s, void* ws,
                 size_t ws_bytes, hipStream_t hs) {
  if (!s || !wdev || !x || !y || !ws) return FB_ERR_NULL;
  const int cus = device_cus();
  int st = mx_gemv_check(s, cus);
  if (st != FB_OK) return st;
  if (!aligned16(wdev) || !aligned16(x) || (reinterpret_cast<uintptr_t>(y) & 3u) ||
      (reinterpret_cast<uintptr_t>(ws) & 255u))
    return FB_ERR_ALIGN;
  const size_t need = mx_split_bytes(s->B, s->K);
  if (ws_bytes < need) return FB_ERR_WORKSPACE;
  st = launch_mx_split(x, ws, s, hs);
  if (st != FB_OK) return st;
  uint8_t* w8 = static_cast<uint8_t*>(ws);
  return gemv_mx_split_run(wdev, w8, y, s, cus, w8 + need, ws_bytes - need, hs);
}

#ifdef FB_PHASE_TRACE
// The launch floor of a GEMV plan (diagnostic library only): a kernel that does nothing, with
// the GEMV's argument block, grid, waves per workgroup and dynamic LDS, holding VG VGPRs (the
// count of the GEMV kernel it stands in for: 183 for the 8-wave GF4 batch-1 kernels, 92 for
// the E2M1 ones), so the same number of its workgroups fit a CU.  Its traced duration and its
// back-to-back rate are what a call of that plan costs before any work.
template <int NW, int VG>
__global__ __launch_bounds__(NW * 64) void floor_kernel(
    const uint8_t* __restrict__ w, const void* __restrict__ x, int K, int Bin, int SPL, int GS,
    int tq, int tr, unsigned spl_m, int S, int fwht_block, int RS, float fwht_scale,
    void* __restrict__ y, int N, int ydt) {
  extern __shared__ __align__(16) uint8_t lds[];
  if constexpr (VG == 183)
    asm volatile("v_mov_b32 v182, 0" ::: "v182");
  else
    asm volatile("v_mov_b32 v91, 0" ::: "v91");
  // never true for a real launch (N >= 1): keeps the arguments and the LDS live
  if (N < 0 && threadIdx.x == 0)
    static_cast<uint8_t*>(y)[blockIdx.x] = lds[threadIdx.x] + w[K] + static_cast<const uint8_t*>(x)[Bin];
}

template <int NW, int VG>
int launch_floor(const fb_shape_t* s, const Plan& pl, hipStream_t stream) {
  auto kern = floor_kernel<NW, VG>;
  static std::atomic<bool> attr_set{false};  // diagnostic library: the first device only
  if (!attr_set.load(std::memory_order_acquire)) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kLdsLimit) != hipSuccess)
      return FB_ERR_HIP;
    attr_set.store(true, std::memory_order_release);
  }
  hipLaunchKernelGGL(kern, dim3(pl.grid), dim3(NW * 64), pl.lds, stream, nullptr, nullptr, s->K,
                     s->B, pl.SPL, pl.GS, pl.tq, pl.tr, div_magic(pl.SPL), pl.S, s->fwht_block,
                     x_row_stride(pl.SPL * 4), fwht_scale(s->fwht_block), nullptr, s->N,
                     s->y_dtype);
  return hipGetLastError() == hipSuccess ? FB_OK : FB_ERR_HIP;
}

// The fill rate of x staging alone (diagnostic library only): every workgroup reads the same
// xbytes of x in 16-byte chunks through a buffer resource, XP per thread, the way the GEMV's
// x preload does, writes them to LDS and meets at a barrier; no weight stream runs beside it.
// Each wave records s_memrealtime (100 MHz) at its start, after its loads are issued, after they
// have arrived and after the barrier, at ts[((blockIdx.x * NT / 64) + wave) * 4 + i], for the
// last of `passes` rounds (a second round reads x that the first left in the caches).
template <int NT, int XP>
__global__ __launch_bounds__(NT) void xfill_kernel(const uint8_t* __restrict__ x, int xbytes,
                                                   int passes, unsigned long long* __restrict__ ts) {
  extern __shared__ __align__(16) uint8_t lds[];
  const rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(x), (short)0, xbytes,
                                                      kRsrcWord3);
  const int n = xbytes / 16;
  unsigned long long t[4];
  t[0] = __builtin_amdgcn_s_memrealtime();
  for (int p = 0; p < passes; ++p) {
    u32x4 v[XP];
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      const int c = threadIdx.x + j * NT;
      if (c < n)
        v[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, c * 16, 0, 0));
    }
    t[1] = __builtin_amdgcn_s_memrealtime();
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      const int c = threadIdx.x + j * NT;
      if (c < n) *reinterpret_cast<u32x4*>(lds + (c & 8191) * 16) = v[j];
    }
    __builtin_amdgcn_s_waitcnt(0);
    t[2] = __builtin_amdgcn_s_memrealtime();
    __syncthreads();
    t[3] = __builtin_amdgcn_s_memrealtime();
  }
  if ((threadIdx.x & 63) == 0) {
    unsigned long long* o = ts + ((size_t)blockIdx.x * (NT / 64) + (threadIdx.x >> 6)) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = t[i];
  }
}

template <int NT, int XP>
int launch_xfill(const void* x, int xbytes, int passes, int grid, void* ts, hipStream_t stream) {
  auto kern = xfill_kernel<NT, XP>;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                          hipFuncAttributeMaxDynamicSharedMemorySize, kLdsLimit) != hipSuccess)
    return FB_ERR_HIP;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(NT), 8192 * 16, stream,
                     static_cast<const uint8_t*>(x), xbytes, passes,
                     static_cast<unsigned long long*>(ts));
  return hipGetLastError() == hipSuccess ? FB_OK : FB_ERR_HIP;
}

// The launch floor of the native FP4 path's split (diagnostic library only): a kernel with
// mx_split_kernel's grid, block and arguments that does nothing.  fb_phase_mx_floor launches
// it and then the GEMV on a split made beforehand, so its time per call against
// fb_gemv_mx_presplit's is what a separate split launch costs before any work.
__global__ __launch_bounds__(64) void split_floor_kernel(const uint16_t* __restrict__ x,
                                                         uint8_t* __restrict__ out, int n8,
                                                         size_t sc_off) {
  // never true for a real launch (n8 >= 16): keeps the arguments live
  if (n8 < 0 && threadIdx.x == 0) out[blockIdx.x] = (uint8_t)x[sc_off];
}
#endif

// Scratch of the allocation-free entry point: a file-scope device array (one per GPU the
// library runs on, alive until the process ends).  Host code never uses the array's name as
// an address: the device address comes from hipGetSymbolAddress, once per device.
constexpr size_t kScratchBytes = size_t(1) << 20;
__device__ __align__(256) uint8_t scratch[kScratchBytes];
std::atomic<void*> g_scratch[kMaxDevices];

// The scratch's device address on the current device (nullptr on failure).
void* scratch_ptr(int dev) {
  if (dev < 0 || dev >= kMaxDevices) return nullptr;
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p) return p;
  void* q = nullptr;
  if (hipGetSymbolAddress(&q, HIP_SYMBOL(scratch)) != hipSuccess || !q) return nullptr;
  g_scratch[dev].store(q, std::memory_order_release);
  return q;
}
#endif  // FB_GEMV_ILP_TU

}  // namespace

#ifdef FB_GEMV_ILP_TU
namespace fb_ilp {
// The 8-wave E2M1 kernels of batches 2-16 at x preload depth xp (4, 8 or 16).
template <int XDT, int MODE>
int launch_e2m1_batch8(const void* wdev, const void* x, void* y, const fb_shape_t* s,
                       const Plan& pl, int xp, hipStream_t stream) {
  if (xp == 4) return launch_gemv<FB_FMT_E2M1, XDT, MODE, kWaves / 2, 4>(wdev, x, y, s, pl, stream);
  if (xp == 8) return launch_gemv<FB_FMT_E2M1, XDT, MODE, kWaves / 2, 8>(wdev, x, y, s, pl, stream);
  return launch_gemv<FB_FMT_E2M1, XDT, MODE, kWaves / 2, 16>(wdev, x, y, s, pl, stream);
}

int launch(int fmt, int xdt, int mode, const void* wdev, const void* x, void* y,
           const fb_shape_t* s, int grid, int SPL, int GS, int tq, int tr, int S, size_t lds,
           int xp, hipStream_t stream) {
  Plan pl;
  pl.grid = grid;
  pl.SPL = SPL;
  pl.GS = GS;
  pl.tq = tq;
  pl.tr = tr;
  pl.S = S;
  pl.lds = lds;
  pl.xp = xp;
  pl.nw = kWaves / 2;
  if (mode == kRot1) {  // a rotation takes fp16 x (and preloads its own way)
    if (xdt != FB_DT_F16) return FB_ERR_DTYPE;
    return fmt == FB_FMT_GF4
               ? launch_gemv<FB_FMT_GF4, FB_DT_F16, kRot1, kWaves / 2, 4>(wdev, x, y, s, pl, stream)
               : launch_gemv<FB_FMT_E2M1, FB_DT_F16, kRot1, kWaves / 2, 4>(wdev, x, y, s, pl, stream);
  }
  if (mode == kRotDA) {
    if (xdt != FB_DT_F16) return FB_ERR_DTYPE;
    return fmt == FB_FMT_GF4
               ? launch_gemv<FB_FMT_GF4, FB_DT_F16, kRotDA, kWaves / 2, 4>(wdev, x, y, s, pl, stream)
               : launch_gemv<FB_FMT_E2M1, FB_DT_F16, kRotDA, kWaves / 2, 4>(wdev, x, y, s, pl, stream);
  }
  if (mode == kRotDAall) {
    if (xdt != FB_DT_F16) return FB_ERR_DTYPE;
    return fmt == FB_FMT_GF4
               ? launch_gemv<FB_FMT_GF4, FB_DT_F16, kRotDAall, kWaves / 2, 4>(wdev, x, y, s, pl, stream)
               : launch_gemv<FB_FMT_E2M1, FB_DT_F16, kRotDAall, kWaves / 2, 4>(wdev, x, y, s, pl, stream);
  }
  if (mode == kSpanX) {
    if (fmt == kFmtMx)
      return xp == 2 ? launch_gemv<kFmtMx, FB_DT_BF16, kSpanX, kWaves / 2, 2>(wdev, x, y, s, pl, stream)
           : xp == 4 ? launch_gemv<kFmtMx, FB_DT_BF16, kSpanX, kWaves / 2, 4>(wdev, x, y, s, pl, stream)
                     : launch_gemv<kFmtMx, FB_DT_BF16, kSpanX, kWaves / 2, 8>(wdev, x, y, s, pl, stream);
    if (fmt == FB_FMT_GF4) {
      if (xdt != FB_DT_F16) return FB_ERR_DTYPE;
      return xp == 2 ? launch_gemv<FB_FMT_GF4, FB_DT_F16, kSpanX, kWaves / 2, 2>(wdev, x, y, s, pl, stream)
           : xp == 4 ? launch_gemv<FB_FMT_GF4, FB_DT_F16, kSpanX, kWaves / 2, 4>(wdev, x, y, s, pl, stream)
                     : launch_gemv<FB_FMT_GF4, FB_DT_F16, kSpanX, kWaves / 2, 8>(wdev, x, y, s, pl, stream);
    }
    if (xdt == FB_DT_BF16)
      return xp == 2 ? launch_gemv<FB_FMT_E2M1, FB_DT_BF16, kSpanX, kWaves / 2, 2>(wdev, x, y, s, pl, stream)
           : xp == 4 ? launch_gemv<FB_FMT_E2M1, FB_DT_BF16, kSpanX, kWaves / 2, 4>(wdev, x, y, s, pl, stream)
                     : launch_gemv<FB_FMT_E2M1, FB_DT_BF16, kSpanX, kWaves / 2, 8>(wdev, x, y, s, pl, stream);
    return xp == 2 ? launch_gemv<FB_FMT_E2M1, FB_DT_F16, kSpanX, kWaves / 2, 2>(wdev, x, y, s, pl, stream)
         : xp == 4 ? launch_gemv<FB_FMT_E2M1, FB_DT_F16, kSpanX, kWaves / 2, 4>(wdev, x, y, s, pl, stream)
                   : launch_gemv<FB_FMT_E2M1, FB_DT_F16, kSpanX, kWaves / 2, 8>(wdev, x, y, s, pl, stream);
  }
  if (mode == kSplitK) {
    pl.P = S;
    if (fmt == FB_FMT_GF4)
      return xp == 4 ? launch_gemv<FB_FMT_GF4, FB_DT_F16, kSplitK, kWaves / 2, 4>(wdev, x, y, s, pl, stream)
           : xp == 8 ? launch_gemv<FB_FMT_GF4, FB_DT_F16, kSplitK, kWaves / 2, 8>(wdev, x, y, s, pl, stream)
                     : launch_gemv<FB_FMT_GF4, FB_DT_F16, kSplitK, kWaves / 2, 16>(wdev, x, y, s, pl, stream);
    if (xdt == FB_DT_BF16)
      return launch_e2m1_batch8<FB_DT_BF16, kSplitK>(wdev, x, y, s, pl, xp, stream);
    return launch_e2m1_batch8<FB_DT_F16, kSplitK>(wdev, x, y, s, pl, xp, stream);
  }
  if ((mode == kSliced || mode == kFlat) && fmt == kFmtMx) {
    if (mode == kSliced)
      return xp == 4 ? launch_gemv<kFmtMx, FB_DT_BF16, kSliced, kWaves / 2, 4>(wdev, x, y, s, pl, stream)
           : xp == 8 ? launch_gemv<kFmtMx, FB_DT_BF16, kSliced, kWaves / 2, 8>(wdev, x, y, s, pl, stream)
                     : launch_gemv<kFmtMx, FB_DT_BF16, kSliced, kWaves / 2, 16>(wdev, x, y, s, pl, stream);
    return xp == 4 ? launch_gemv<kFmtMx, FB_DT_BF16, kFlat, kWaves / 2, 4>(wdev, x, y, s, pl, stream)
         : xp == 8 ? launch_gemv<kFmtMx, FB_DT_BF16, kFlat, kWaves / 2, 8>(wdev, x, y, s, pl, stream)
                   : launch_gemv<kFmtMx, FB_DT_BF16, kFlat, kWaves / 2, 16>(wdev, x, y, s, pl, stream);
  }
  if ((mode == kSliced || mode == kFlat) && fmt == FB_FMT_E2M1) {
    if (xdt == FB_DT_BF16)
      return mode == kSliced ? launch_e2m1_batch8<FB_DT_BF16, kSliced>(wdev, x, y, s, pl, xp, stream)
                             : launch_e2m1_batch8<FB_DT_BF16, kFlat>(wdev, x, y, s, pl, xp, stream);
    return mode == kSliced ? launch_e2m1_batch8<FB_DT_F16, kSliced>(wdev, x, y, s, pl, xp, stream)
                           : launch_e2m1_batch8<FB_DT_F16, kFlat>(wdev, x, y, s, pl, xp, stream);
  }
  if (mode == kSliced) {
    if (fmt != FB_FMT_GF4 || xdt != FB_DT_F16) return FB_ERR_DTYPE;
    if (xp == 4) return launch_gemv<FB_FMT_GF4, FB_DT_F16, kSliced, kWaves / 2, 4>(wdev, x, y, s, pl, stream);
    if (xp == 8) return launch_gemv<FB_FMT_GF4, FB_DT_F16, kSliced, kWaves / 2, 8>(wdev, x, y, s, pl, stream);
    return launch_gemv<FB_FMT_GF4, FB_DT_F16, kSliced, kWaves / 2, 16>(wdev, x, y, s, pl, stream);
  }
  if (mode == kFlat) {  // GF4 at batch 2-16 in one K-slice (E2M1: above)
    if (fmt != FB_FMT_GF4 || xdt != FB_DT_F16) return FB_ERR_DTYPE;
    if (xp == 4) return launch_gemv<FB_FMT_GF4, FB_DT_F16, kFlat, kWaves / 2, 4>(wdev, x, y, s, pl, stream);
    if (xp == 8) return launch_gemv<FB_FMT_GF4, FB_DT_F16, kFlat, kWaves / 2, 8>(wdev, x, y, s, pl, stream);
    return launch_gemv<FB_FMT_GF4, FB_DT_F16, kFlat, kWaves / 2, 16>(wdev, x, y, s, pl, stream);
  }
  // kFlat1: GF4 with fp16 x, E2M1 with fp16 or bf16 x
  if (xp >= 8) {
    if (fmt == FB_FMT_GF4)
      return launch_gemv<FB_FMT_GF4, FB_DT_F16, kFlat1, kWaves / 2, 8>(wdev, x, y, s, pl, stream);
    if (xdt == FB_DT_BF16)
      return launch_gemv<FB_FMT_E2M1, FB_DT_BF16, kFlat1, kWaves / 2, 8>(wdev, x, y, s, pl, stream);
    return launch_gemv<FB_FMT_E2M1, FB_DT_F16, kFlat1, kWaves / 2, 8>(wdev, x, y, s, pl, stream);
  }
  if (fmt == FB_FMT_GF4)
    return launch_gemv<FB_FMT_GF4, FB_DT_F16, kFlat1, kWaves / 2, 4>(wdev, x, y, s, pl, stream);
  if (xdt == FB_DT_BF16)
    return launch_gemv<FB_FMT_E2M1, FB_DT_BF16, kFlat1, kWaves / 2, 4>(wdev, x, y, s, pl, stream);
  return launch_gemv<FB_FMT_E2M1, FB_DT_F16, kFlat1, kWaves / 2, 4>(wdev, x, y, s, pl, stream);
}
}  // namespace fb_ilp
#else

extern "C" {

int fb_gemv_noalloc(const void* wdev, const void* x, void* y, const fb_shape_t* s,
                    void* stream) {
  if (!s) return FB_ERR_NULL;
  const int st = fb_validate(s);
  if (st != FB_OK) return st;
  const size_t need = rot_once_bytes(s);
  if (need > kScratchBytes) return FB_ERR_SCRATCH;
  // the rotation's x' and, where they fit after it, the split-K parts' sums (else the
  // K-slices run in turn, as without a workspace)
  void* ws = nullptr;
  if (fb_workspace_bytes(s)) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return FB_ERR_HIP;
    ws = scratch_ptr(dev);
    if (!ws) return FB_ERR_HIP;
  }
  return gemv_impl(wdev, x, y, s, ws, ws ? kScratchBytes : 0, static_cast<hipStream_t>(stream));
}

size_t fb_workspace_bytes(const fb_shape_t* s) {
  if (fb_validate(s) != FB_OK) return 0;
  const size_t rot = rot_once_bytes(s);
  fb_shape_t u = *s;
  if (rot) u.fwht_block = 0;  // the GEMV after the rotation is unrotated
  return rot + splitk_bytes(&u, splitk_parts(&u, device_cus(), nullptr));
}

int fb_gemv(const void* wdev, const void* x, void* y, const fb_shape_t* s, void* ws,
            size_t ws_bytes, void* stream) {
  return gemv_impl(wdev, x, y, s, ws, ws_bytes, static_cast<hipStream_t>(stream));
}

int fb_dequant(const void* wdev, void* w_out, int32_t out_dtype, const fb_shape_t* s,
               void* stream) {
  if (!s || !wdev || !w_out) return FB_ERR_NULL;
  int st = fb_validate(s);
  if (st != FB_OK) return st;
  if (out_dtype != FB_DT_F32 && out_dtype != FB_DT_F16 && out_dtype != FB_DT_BF16)
    return FB_ERR_DTYPE;
  if (!aligned16(wdev)) return FB_ERR_ALIGN;
  const int64_t items = (int64_t)s->N * (s->K / 128);  // < 2^31 (fb_validate)
  const int grid = (int)((items + 255) / 256);
  hipStream_t hs = static_cast<hipStream_t>(stream);
  if (s->fmt == FB_FMT_GF4)
    hipLaunchKernelGGL(dequant_kernel<FB_FMT_GF4>, dim3(grid), dim3(256), 0, hs,
                       static_cast<const uint8_t*>(wdev), w_out, s->N, s->K, out_dtype);
  else
    hipLaunchKernelGGL(dequant_kernel<FB_FMT_E2M1>, dim3(grid), dim3(256), 0, hs,
                       static_cast<const uint8_t*>(wdev), w_out, s->N, s->K, out_dtype);
  return hipGetLastError() == hipSuccess ? FB_OK : FB_ERR_HIP;
}

size_t fb_mx_split_bytes(const fb_shape_t* s) {
  if (!s || mx_check(s) != FB_OK) return 0;
  return mx_split_bytes(s->B, s->K);
}

int fb_mx_split(const void* x, void* out, const fb_shape_t* s, void* stream) {
  if (!s || !x || !out) return FB_ERR_NULL;
  const int st = mx_check(s);
  if (st != FB_OK) return st;
  if (!aligned16(x) || (reinterpret_cast<uintptr_t>(out) & 255u)) return FB_ERR_ALIGN;
  return launch_mx_split(x, out, s, static_cast<hipStream_t>(stream));
}

size_t fb_mx_workspace_bytes(const fb_shape_t* s) {
  if (!s || mx_check(s) != FB_OK) return 0;
  fb_shape_t u = *s;
  u.fmt = kFmtMx;
  return mx_split_bytes(s->B, s->K) + splitk_bytes(&u, splitk_parts(&u, device_cus(), nullptr));
}

int fb_gemv_mx(const void* wdev, const void* x, void* y, const fb_shape_t* s, void* ws,
               size_t ws_bytes, void* stream) {
  return gemv_mx_impl(wdev, x, y, s, ws, ws_bytes, static_cast<hipStream_t>(stream));
}

int fb_gemv_mx_presplit(const void* wdev, const void* xs, void* y, const fb_shape_t* s,
                        void* ws, size_t ws_bytes, void* stream) {
  if (!s || !wdev || !xs || !y) return FB_ERR_NULL;
  const int cus = device_cus();
  const int st = mx_gemv_check(s, cus);
  if (st != FB_OK) return st;
  if (!aligned16(wdev) || (reinterpret_cast<uintptr_t>(xs) & 255u) ||
      (reinterpret_cast<uintptr_t>(y) & 3u))
    return FB_ERR_ALIGN;
  if (ws && (reinterpret_cast<uintptr_t>(ws) & 255u)) ws = nullptr;  // misaligned: unused
  if (!ws) ws_bytes = 0;
  return gemv_mx_split_run(wdev, xs, y, s, cus, ws, ws_bytes, static_cast<hipStream_t>(stream));
}

#ifdef FB_PHASE_TRACE
// fb_gemv_mx_presplit after an empty kernel with the split's launch shape (diagnostic
// library; see split_floor_kernel).  xs: a split made beforehand, as for the presplit call.
int fb_phase_mx_floor(const void* wdev, const void* xs, void* y, const fb_shape_t* s, void* ws,
                      size_t ws_bytes, void* stream) {
  if (!s || !wdev || !xs || !y) return FB_ERR_NULL;
  const int st = mx_gemv_check(s, device_cus());
  if (st != FB_OK) return st;
  const int n8 = s->B * (s->K / 8);
  hipLaunchKernelGGL(split_floor_kernel, dim3((n8 + 63) / 64), dim3(64), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(xs),
                     static_cast<uint8_t*>(ws ? ws : y), n8, mx_scale_offset(s->B, s->K));
  if (hipGetLastError() != hipSuccess) return FB_ERR_HIP;
  return fb_gemv_mx_presplit(wdev, xs, y, s, ws, ws_bytes, stream);
}
#endif

size_t fb_mx_presplit_workspace_bytes(const fb_shape_t* s) {
  if (!s || mx_check(s) != FB_OK) return 0;
  fb_shape_t u = *s;
  u.fmt = kFmtMx;
  return splitk_bytes(&u, splitk_parts(&u, device_cus(), nullptr));
}

#ifdef FB_PHASE_TRACE
// Diagnostic library only.  The buffer (device memory, `entries` 64-bit values) that the
// following GEMV launches write their phase timestamps to, or null for none.  A launch
// whose grid needs more entries writes nothing.  Not for concurrent use.
int fb_phase_trace_set(void* buf, size_t entries) {
  g_phase_host = static_cast<unsigned long long*>(buf);
  g_phase_entries = buf ? entries : 0;
  return FB_OK;
}

// The launch plan fb_gemv uses for a shape on the current device, given a workspace of
// fb_workspace_bytes(s): workgroups (per K-part), waves per workgroup, K-slices (split-K:
// parts), row tiles per workgroup (the first tr take one more), and the split-K part count
// (0: the slices in turn).
int fb_phase_plan(const fb_shape_t* s, int* grid, int* waves, int* slices, int* tq, int* tr,
                  int* parts) {
  if (!s || !grid || !waves || !slices || !tq || !tr || !parts) return FB_ERR_NULL;
  const int st = fb_validate(s);
  if (st != FB_OK) return st;
  Plan pl;
  if (!splitk_parts(s, device_cus(), &pl) && !make_plan(s, device_cus(), pl)) return FB_ERR_LDS;
  *grid = pl.grid;
  *waves = pl.nw;
  *slices = pl.spanx ? 0 : pl.S;  // 0: kSpanX (each wave stages its own spans)
  *tq = pl.tq;
  *tr = pl.tr;
  *parts = pl.P;
  return FB_OK;
}

// The split-K part count of the following calls (see g_force_parts); not for concurrent use.
int fb_phase_force_parts(int parts) {
  if (parts != 0 && parts != -1 && parts != 2 && parts != 4 && parts != 8) return FB_ERR_SHAPE;
  g_force_parts.store(parts, std::memory_order_relaxed);
  return FB_OK;
}

// Launches xfill_kernel: grid workgroups of `threads` (512 or 1024) threads each read the same
// xbytes (a multiple of 16, at most 256 KiB) of x into LDS, `passes` (1 or 2) times; ts holds
// grid * threads / 64 * 4 timestamps.
int fb_phase_xfill(const void* x, int xbytes, int threads, int passes, int grid, void* ts,
                   void* stream) {
  if (!x || !ts) return FB_ERR_NULL;
  if (xbytes < 16 || xbytes % 16 || xbytes > 256 * 1024 || (threads != 512 && threads != 1024) ||
      passes < 1 || passes > 2 || grid < 1 || grid > 65535)
    return FB_ERR_SHAPE;
  hipStream_t hs = static_cast<hipStream_t>(stream);
  const int per = (xbytes / 16 + threads - 1) / threads;  // chunks per thread
  if (threads == 1024) {
    if (per <= 1) return launch_xfill<1024, 1>(x, xbytes, passes, grid, ts, hs);
    if (per <= 4) return launch_xfill<1024, 4>(x, xbytes, passes, grid, ts, hs);
    if (per <= 8) return launch_xfill<1024, 8>(x, xbytes, passes, grid, ts, hs);
    return launch_xfill<1024, 16>(x, xbytes, passes, grid, ts, hs);
  }
  if (per <= 2) return launch_xfill<512, 2>(x, xbytes, passes, grid, ts, hs);
  if (per <= 8) return launch_xfill<512, 8>(x, xbytes, passes, grid, ts, hs);
  if (per <= 16) return launch_xfill<512, 16>(x, xbytes, passes, grid, ts, hs);
  return launch_xfill<512, 32>(x, xbytes, passes, grid, ts, hs);
}

// Launches floor_kernel with the plan fb_gemv would launch for a batch-1 shape that runs one
// kernel (no workspace): its grid, waves and LDS, and the register count of the GF4 (183) or
// E2M1 (92) 8-wave kernel.
int fb_phase_floor(const fb_shape_t* s, void* stream) {
  if (!s) return FB_ERR_NULL;
  const int st = fb_validate(s);
  if (st != FB_OK) return st;
  Plan pl;
  if (!make_plan(s, device_cus(), pl)) return FB_ERR_LDS;
  hipStream_t hs = static_cast<hipStream_t>(stream);
  const bool gf4 = s->fmt == FB_FMT_GF4;
  if (pl.nw == kWaves / 2)
    return gf4 ? launch_floor<kWaves / 2, 183>(s, pl, hs) : launch_floor<kWaves / 2, 92>(s, pl, hs);
  return launch_floor<kWaves, 92>(s, pl, hs);
}
#endif

}  // extern "C"
#endif  // FB_GEMV_ILP_TU
