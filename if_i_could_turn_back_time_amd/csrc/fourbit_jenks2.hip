// Two-class natural breaks (k = 2 Jenks) over a whole array on the GPU, in O(n) after the
// sort: the reference's weight/bias pruning rule (Linear_Mask / Bias_Mask,
// Python_Jenks_Test/Jenks_Tests/cuda_helpers.py:378-411, kernels :85-118 and :151-184,
// also CUDA_C_Code/include/layers.h:2424-2560).  The reference launches one thread per split
// index, each summing both classes serially (O(n^2)); here the classes' sums come from
// prefix sums, so every split costs a few operations.
//
// Rule (shared with fb_jenks2_host, which computes the same bits on the CPU):
//  1. Sort the values ascending, stable by index (-0.0 and +0.0 are equal).
//  2. c = sorted[n / 2]; d_t = sorted[t] - c and q_t = d_t * d_t in fp64 (the SSD is
//     invariant to the shift; centering keeps the prefix sums free of cancellation).
//  3. Prefix sums of d and q in a fixed association order: sequential within blocks of
//     256 elements (Lx, exclusive), block totals sequential within superblocks of 256
//     blocks (Bx, exclusive), superblock totals sequential (Sx, exclusive, Sx[S] = total);
//     P(i) = (Sx[s] + Bx[b]) + Lx(i).
//  4. For every split i in [0, n): ssd(i) = [i ? Q(i) - P(i)^2 / i : 0]
//     + [(Qt - Q(i)) - (Pt - P(i))^2 / (n - i)]; split 0 is "no split".
//  5. split = the first index of the minimum; the elements at sorted positions >= split
//     are kept; GVF = (ssd(0) - ssd(split)) / (ssd(0) + 1e-8).
// The file is compiled with -ffp-contract=off so no multiply-add is fused: every fp64
// operation rounds as the host's does.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <cstdint>

#include "fourbit.h"

namespace {

constexpr int kBlk = 256;  // elements per block (sequential local sums)
constexpr int kSup = 256;  // blocks per superblock

struct J2Layout {
  int64_t n, nblk, nsup;
  size_t sort_bytes;
  size_t off_keys_in, off_keys_out, off_vals_in, off_vals_out, off_sort;
  size_t off_t1, off_t2, off_bx1, off_bx2, off_u1, off_u2, off_sx1, off_sx2;
  size_t off_bmin, off_bidx, off_smin, off_sidx, off_ssd0, total;
};

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

int j2_layout(int64_t n, J2Layout& L) {
  L.n = n;
  L.nblk = (n + kBlk - 1) / kBlk;
  L.nsup = (L.nblk + kSup - 1) / kSup;
  size_t sort_bytes = 0;
  if (hipcub::DeviceRadixSort::SortPairs(nullptr, sort_bytes, (const float*)nullptr,
                                         (float*)nullptr, (const int*)nullptr, (int*)nullptr,
                                         (int)n, 0, 32, (hipStream_t)0) != hipSuccess)
    return FB_ERR_HIP;
  L.sort_bytes = sort_bytes;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o = align256(o + bytes);
    return at;
  };
  L.off_keys_in = take(4 * (size_t)n);
  L.off_keys_out = take(4 * (size_t)n);
  L.off_vals_in = take(4 * (size_t)n);
  L.off_vals_out = take(4 * (size_t)n);
  L.off_sort = take(sort_bytes);
  L.off_t1 = take(8 * (size_t)L.nblk);
  L.off_t2 = take(8 * (size_t)L.nblk);
  L.off_bx1 = take(8 * (size_t)L.nblk);
  L.off_bx2 = take(8 * (size_t)L.nblk);
  L.off_u1 = take(8 * (size_t)L.nsup);
  L.off_u2 = take(8 * (size_t)L.nsup);
  L.off_sx1 = take(8 * (size_t)(L.nsup + 1));
  L.off_sx2 = take(8 * (size_t)(L.nsup + 1));
  L.off_bmin = take(8 * (size_t)L.nblk);
  L.off_bidx = take(4 * (size_t)L.nblk);
  L.off_smin = take(8 * (size_t)L.nsup);
  L.off_sidx = take(4 * (size_t)L.nsup);
  L.off_ssd0 = take(8);
  L.total = o;
  return FB_OK;
}

// keys: the values with -0.0 made +0.0 (so the radix order treats them as equal and the
// sort keeps their index order); payload: the index.
__global__ void j2_prep(const float* __restrict__ w, float* __restrict__ keys,
                        int* __restrict__ vals, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const float v = w[i];
    keys[i] = v == 0.0f ? 0.0f : v;
    vals[i] = i;
  }
}

template <typename T>
__device__ __forceinline__ double centre(const T* __restrict__ s, int n) {
  return (double)s[n / 2];
}

// The serial sums below keep the fixed association order; what changes between kernels is
// only how the operands reach the thread.  A thread that walks one block reads it in
// 16-value pieces, one contiguous 64-byte read per lane (lanes are a block apart, so
// single-value reads would touch 64 lines per instruction for 4 bytes each).
constexpr int kPiece = 16;

// kPiece values of T (float or double) from 16-byte aligned p, in 16-byte reads.
template <typename T>
__device__ __forceinline__ void load_piece(const T* __restrict__ p, T (&f)[kPiece]) {
  constexpr int kVec = 16 / sizeof(T);
#pragma unroll
  for (int r = 0; r < kPiece / kVec; ++r)
    *reinterpret_cast<uint4*>(f + kVec * r) = reinterpret_cast<const uint4*>(p)[r];
}
template <typename T>
__device__ __forceinline__ void store_piece(T* __restrict__ p, const T (&f)[kPiece]) {
  constexpr int kVec = 16 / sizeof(T);
#pragma unroll
  for (int r = 0; r < kPiece / kVec; ++r)
    reinterpret_cast<uint4*>(p)[r] = *reinterpret_cast<const uint4*>(f + kVec * r);
}

// Block totals of d and q: one thread per block of kBlk sorted values (T: float or double).
template <typename T>
__global__ void j2_block_totals(const T* __restrict__ s, int n, int nblk,
                                double* __restrict__ t1, double* __restrict__ t2) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblk) return;
  const double c = centre(s, n);
  const int i0 = b * kBlk, i1 = min(n, i0 + kBlk);
  double a1 = 0.0, a2 = 0.0;
  int i = i0;
  for (; i + kPiece <= i1; i += kPiece) {
    T f[kPiece];
    load_piece(s + i, f);
#pragma unroll
    for (int e = 0; e < kPiece; ++e) {
      const double d = (double)f[e] - c;
      const double q = d * d;
      a1 = a1 + d;
      a2 = a2 + q;
    }
  }
  for (; i < i1; ++i) {
    const double d = (double)s[i] - c;
    const double q = d * d;
    a1 = a1 + d;
    a2 = a2 + q;
  }
  t1[b] = a1;
  t2[b] = a2;
}

// Exclusive block prefixes within each superblock and the superblock totals: one thread per
// superblock, reading and writing 4 blocks' values at a time.
__global__ void j2_super(const double* __restrict__ t1, const double* __restrict__ t2, int nblk,
                         int nsup, double* __restrict__ bx1, double* __restrict__ bx2,
                         double* __restrict__ u1, double* __restrict__ u2) {
  const int s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s >= nsup) return;
  const int b0 = s * kSup, b1 = min(nblk, b0 + kSup);
  double a1 = 0.0, a2 = 0.0;
  int b = b0;
  for (; b + 4 <= b1; b += 4) {
    double v1[4], v2[4], o1[4], o2[4];
    *reinterpret_cast<double2*>(v1) = reinterpret_cast<const double2*>(t1 + b)[0];
    *reinterpret_cast<double2*>(v1 + 2) = reinterpret_cast<const double2*>(t1 + b)[1];
    *reinterpret_cast<double2*>(v2) = reinterpret_cast<const double2*>(t2 + b)[0];
    *reinterpret_cast<double2*>(v2 + 2) = reinterpret_cast<const double2*>(t2 + b)[1];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o1[e] = a1;
      o2[e] = a2;
      a1 = a1 + v1[e];
      a2 = a2 + v2[e];
    }
    reinterpret_cast<double2*>(bx1 + b)[0] = *reinterpret_cast<double2*>(o1);
    reinterpret_cast<double2*>(bx1 + b)[1] = *reinterpret_cast<double2*>(o1 + 2);
    reinterpret_cast<double2*>(bx2 + b)[0] = *reinterpret_cast<double2*>(o2);
    reinterpret_cast<double2*>(bx2 + b)[1] = *reinterpret_cast<double2*>(o2 + 2);
  }
  for (; b < b1; ++b) {
    bx1[b] = a1;
    bx2[b] = a2;
    a1 = a1 + t1[b];
    a2 = a2 + t2[b];
  }
  u1[s] = a1;
  u2[s] = a2;
}

// Exclusive superblock prefixes; sx[nsup] is the total.  The workgroup stages the superblock
// totals through LDS in chunks; thread 0 runs the sequential sums from there.
constexpr int kTopThreads = 256;
constexpr int kTopChunk = 2048;
__global__ __launch_bounds__(kTopThreads) void j2_top(const double* __restrict__ u1,
                                                      const double* __restrict__ u2, int nsup,
                                                      double* __restrict__ sx1,
                                                      double* __restrict__ sx2) {
  __shared__ double l1[kTopChunk], l2[kTopChunk];
  double a1 = 0.0, a2 = 0.0;
  for (int base = 0; base < nsup; base += kTopChunk) {
    const int m = min(kTopChunk, nsup - base);
    for (int i = threadIdx.x; i < m; i += kTopThreads) {
      l1[i] = u1[base + i];
      l2[i] = u2[base + i];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int i = 0; i < m; ++i) {
        sx1[base + i] = a1;
        sx2[base + i] = a2;
        a1 = a1 + l1[i];
        a2 = a2 + l2[i];
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    sx1[nsup] = a1;
    sx2[nsup] = a2;
  }
}

// The SSD of every split of one block, and the block's first minimum; with `out`, every
// split's SSD is also written there, rounded to T.
template <typename T>
__global__ void j2_ssd(const T* __restrict__ s, int n, int nblk, int nsup,
                       const double* __restrict__ bx1, const double* __restrict__ bx2,
                       const double* __restrict__ sx1, const double* __restrict__ sx2,
                       double* __restrict__ bmin, int* __restrict__ bidx,
                       double* __restrict__ ssd0, T* __restrict__ out) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblk) return;
  const double c = centre(s, n);
  const int sup = b / kSup;
  const double base1 = sx1[sup] + bx1[b], base2 = sx2[sup] + bx2[b];
  const double pt = sx1[nsup], qt = sx2[nsup];
  const int i0 = b * kBlk, i1 = min(n, i0 + kBlk);
  double l1 = 0.0, l2 = 0.0;
  double best = 0.0;
  int arg = -1;
  auto step = [&](int i, T v) -> double {
    const double p = base1 + l1, q = base2 + l2;
    const double left = i == 0 ? 0.0 : q - (p * p) / (double)i;
    const double rp = pt - p;
    const double right = (qt - q) - (rp * rp) / (double)(n - i);
    const double sv = left + right;
    if (arg < 0 || sv < best) {
      best = sv;
      arg = i;
    }
    if (i == 0) *ssd0 = sv;
    const double d = (double)v - c;
    const double dq = d * d;
    l1 = l1 + d;
    l2 = l2 + dq;
    return sv;
  };
  int i = i0;
  for (; i + kPiece <= i1; i += kPiece) {
    T f[kPiece], o[kPiece];
    load_piece(s + i, f);
#pragma unroll
    for (int e = 0; e < kPiece; ++e) o[e] = (T)step(i + e, f[e]);
    if (out) store_piece(out + i, o);
  }
  for (; i < i1; ++i) {
    const double sv = step(i, s[i]);
    if (out) out[i] = (T)sv;
  }
  bmin[b] = best;
  bidx[b] = arg;
}

// (value, index) pairs in the order "first index of the minimum": a smaller value wins, an
// equal value goes to the smaller index.  Over indices that increase along the array this
// is exactly the sequential scan with strict <, so a tree of it gives the same winner.
__device__ __forceinline__ void lex_min(double& v, int& i, double v2, int i2) {
  if (v2 < v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

__device__ __forceinline__ void wave_lex_min(double& v, int& i) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const double v2 = __shfl_xor(v, m, 64);
    const int i2 = __shfl_xor(i, m, 64);
    lex_min(v, i, v2, i2);
  }
}

// First minimum over the blocks of each superblock: one wave per superblock.
__global__ __launch_bounds__(64) void j2_min_super(const double* __restrict__ bmin,
                                                   const int* __restrict__ bidx, int nblk,
                                                   int nsup, double* __restrict__ smin,
                                                   int* __restrict__ sidx) {
  const int s = blockIdx.x;
  const int b0 = s * kSup, b1 = min(nblk, b0 + kSup);
  double best = bmin[b0];
  int arg = bidx[b0];
  for (int b = b0 + (int)threadIdx.x; b < b1; b += 64) lex_min(best, arg, bmin[b], bidx[b]);
  wave_lex_min(best, arg);
  if (threadIdx.x == 0) {
    smin[s] = best;
    sidx[s] = arg;
  }
}

constexpr int kFinalThreads = 256;
__global__ __launch_bounds__(kFinalThreads) void j2_final(const double* __restrict__ smin,
                                                          const int* __restrict__ sidx, int nsup,
                                                          const double* __restrict__ ssd0,
                                                          int64_t* __restrict__ split,
                                                          double* __restrict__ gvf) {
  __shared__ double lv[kFinalThreads / 64];
  __shared__ int li[kFinalThreads / 64];
  double best = smin[0];
  int arg = sidx[0];
  for (int s = threadIdx.x; s < nsup; s += kFinalThreads) lex_min(best, arg, smin[s], sidx[s]);
  wave_lex_min(best, arg);
  if ((threadIdx.x & 63) == 0) {
    lv[threadIdx.x >> 6] = best;
    li[threadIdx.x >> 6] = arg;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kFinalThreads / 64; ++w) lex_min(best, arg, lv[w], li[w]);
    *split = arg;
    const double t = *ssd0;
    *gvf = (t - best) / (t + 1e-8);
  }
}

// keep[i] = 1 when w[i] sits at a sorted position >= split.  With t the value at position
// split: every value above t is kept and every value below is not; values equal to t sit in
// index order (the sort is stable), so of those the ones at index >= order[split] are kept.
// A streaming pass over w, not a scatter through the permutation.  (-0.0 == +0.0 as floats,
// as in the sort's keys.)
__global__ void j2_mask(const float* __restrict__ w, const float* __restrict__ skeys,
                        const int* __restrict__ order, int n, const int64_t* __restrict__ split,
                        uint8_t* __restrict__ keep) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t sp = *split;
  const float t = skeys[sp];
  const int it = order[sp];
  const float v = w[i];
  keep[i] = (v > t || (v == t && i >= it)) ? 1 : 0;
}

int grid_of(int64_t items, int threads) { return (int)((items + threads - 1) / threads); }

// ---------------------------------------------------------------------------------
// Every filter of a convolution weight on its own (the reference's Conv_Mask,
// cuda_helpers.py:333-376, over its kernel at :219-255), filters of n <= FB_JENKS2_FILTER_MAX
// values:
//  - The stable ascending order by counting: the rank of value i is the number of values
//    that sort before it, (w_j < w_i) or (w_j == w_i and j < i), so -0.0 and +0.0 tie and
//    keep their index order, as the host's stable sort does.  No sorting network, no
//    workspace.
//  - The fp64 sums of the rule above in one lane per filter, in the host's association
//    order: with n <= 1024 there are at most 4 blocks and one superblock, and every
//    addition the host makes (zeros included) is made here in the same order.
// Many small filters (n <= kLaneFilterMax: 1x1 to 5x5, the common conv kernels; at least
// kLaneFilterMin of them) run one filter per lane, 256 per workgroup.  Otherwise each filter
// has a one-wave workgroup (so that a few filters still spread over the CUs), each lane
// ranking its up to 16 values against the filter, read once per value from LDS.
// ---------------------------------------------------------------------------------
constexpr int kFilterMax = FB_JENKS2_FILTER_MAX;
constexpr int kLaneFilterMax = 25;  // 256 filters x 10 bytes per value fit 64 KiB of LDS
constexpr int kLaneFilterMin = 1024;  // 4 workgroups: fewer filters spread better one per wave
static_assert(kFilterMax <= 4 * kBlk, "one superblock of at most 4 blocks");

// The split and GVF of one sorted filter (srt, n values), in the host's order.
__device__ void filter_split(const float* srt, int n, int& arg_out, double& gvf_out) {
  const int nblk = (n + kBlk - 1) / kBlk;
  const double c = (double)srt[n / 2];
  double t1[4], t2[4], bx1[4], bx2[4];
  for (int b = 0; b < nblk; ++b) {  // block totals
    double a1 = 0.0, a2 = 0.0;
    for (int i = b * kBlk; i < min(n, b * kBlk + kBlk); ++i) {
      const double d = (double)srt[i] - c;
      const double q = d * d;
      a1 = a1 + d;
      a2 = a2 + q;
    }
    t1[b] = a1;
    t2[b] = a2;
  }
  double u1, u2;  // the one superblock: exclusive block offsets, then its total
  {
    double a1 = 0.0, a2 = 0.0;
    for (int b = 0; b < nblk; ++b) {
      bx1[b] = a1;
      bx2[b] = a2;
      a1 = a1 + t1[b];
      a2 = a2 + t2[b];
    }
    u1 = a1;
    u2 = a2;
  }
  const double sx1 = 0.0, sx2 = 0.0;  // the superblocks' exclusive offset (one superblock)
  const double pt = 0.0 + u1, qt = 0.0 + u2;
  double best = 0.0, ssd0 = 0.0;
  int arg = -1;
  for (int b = 0; b < nblk; ++b) {
    const double base1 = sx1 + bx1[b], base2 = sx2 + bx2[b];
    double l1 = 0.0, l2 = 0.0;
    for (int i = b * kBlk; i < min(n, b * kBlk + kBlk); ++i) {
      const double p = base1 + l1, q = base2 + l2;
      const double left = i == 0 ? 0.0 : q - (p * p) / (double)i;
      const double rp = pt - p;
      const double right = (qt - q) - (rp * rp) / (double)(n - i);
      const double val = left + right;
      if (arg < 0 || val < best) {
        best = val;
        arg = i;
      }
      if (i == 0) ssd0 = val;
      const double d = (double)srt[i] - c;
      const double dq = d * d;
      l1 = l1 + d;
      l2 = l2 + dq;
    }
  }
  arg_out = arg;
  gvf_out = (ssd0 - best) / (ssd0 + 1e-8);
}

// The same sums for a wave: one lane stores P(i), Q(i) (the class-0 sums before value i, in
// the host's association order) and the totals; the SSD of every split (two fp64 divisions
// each, the bulk of the work) is then evaluated by all lanes, and the first minimum found by
// a (value, index) reduction, which picks what the host's sequential strict-< scan picks.
__device__ void filter_prefix(const float* srt, int n, double* P, double* Q, double* tot) {
  const int nblk = (n + kBlk - 1) / kBlk;
  const double c = (double)srt[n / 2];
  double t1[4], t2[4], bx1[4], bx2[4];
  for (int b = 0; b < nblk; ++b) {
    double a1 = 0.0, a2 = 0.0;
    for (int i = b * kBlk; i < min(n, b * kBlk + kBlk); ++i) {
      const double d = (double)srt[i] - c;
      const double q = d * d;
      a1 = a1 + d;
      a2 = a2 + q;
    }
    t1[b] = a1;
    t2[b] = a2;
  }
  double u1, u2;
  {
    double a1 = 0.0, a2 = 0.0;
    for (int b = 0; b < nblk; ++b) {
      bx1[b] = a1;
      bx2[b] = a2;
      a1 = a1 + t1[b];
      a2 = a2 + t2[b];
    }
    u1 = a1;
    u2 = a2;
  }
  const double sx1 = 0.0, sx2 = 0.0;
  tot[0] = 0.0 + u1;
  tot[1] = 0.0 + u2;
  for (int b = 0; b < nblk; ++b) {
    const double base1 = sx1 + bx1[b], base2 = sx2 + bx2[b];
    double l1 = 0.0, l2 = 0.0;
    for (int i = b * kBlk; i < min(n, b * kBlk + kBlk); ++i) {
      P[i] = base1 + l1;
      Q[i] = base2 + l2;
      const double d = (double)srt[i] - c;
      const double dq = d * d;
      l1 = l1 + d;
      l2 = l2 + dq;
    }
  }
}

// n <= kLaneFilterMax: thread t of the workgroup does filter blockIdx.x * 256 + t.  LDS: the
// values, their sorted copy, the positions (bytes) and the mask (bytes), 256 filters each.
__global__ __launch_bounds__(256) void j2_filters_lane(const float* __restrict__ w, int64_t nf,
                                                       int n, uint8_t* __restrict__ keep,
                                                       int* __restrict__ split,
                                                       double* __restrict__ gvf) {
  extern __shared__ float lds_f[];
  const int64_t f0 = (int64_t)blockIdx.x * 256;
  const int cnt = (int)min((int64_t)256, nf - f0);
  float* v = lds_f;
  float* srt = v + 256 * n;
  uint8_t* ord = reinterpret_cast<uint8_t*>(srt + 256 * n);
  uint8_t* mk = ord + 256 * n;
  for (int e = threadIdx.x; e < cnt * n; e += 256) v[e] = w[f0 * n + e];  // coalesced
  __syncthreads();
  const int t = threadIdx.x;
  if (t < cnt) {
    const float* vf = v + t * n;
    float* sf = srt + t * n;
    uint8_t* of = ord + t * n;
    for (int i = 0; i < n; ++i) {
      const float x = vf[i];
      int r = 0;
#pragma unroll 5
      for (int j = 0; j < n; ++j) {
        const float y = vf[j];
        r += (int)(y < x) | ((int)(y == x) & (int)(j < i));
      }
      sf[r] = x;
      of[r] = (uint8_t)i;
    }
    int arg;
    double g;
    filter_split(sf, n, arg, g);
    split[f0 + t] = arg;
    gvf[f0 + t] = g;
    for (int r = 0; r < n; ++r) mk[t * n + of[r]] = r >= arg ? 1 : 0;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < cnt * n; e += 256) keep[f0 * n + e] = mk[e];  // coalesced
}

// LDS of the one-wave filter kernel: the values and their sorted copy (fp32), the positions
// (int16, padded to 8 bytes), then the class sums P, Q and the two totals (fp64).
__host__ __device__ inline size_t wave_sums_offset(int n) {
  return ((size_t)n * 8 + (size_t)n * 2 + 7) & ~size_t(7);
}
__host__ __device__ inline size_t wave_lds_bytes(int n) {
  return wave_sums_offset(n) + (size_t)n * 16 + 16;
}

// One filter per one-wave workgroup (blockIdx.x).  Each lane keeps its values l, l + 64, ...
// (KC of them, KC = n / 64 rounded up to a power of two, at most 16) in registers and counts,
// for each of them, the values that sort before it, reading every value of the filter once
// from LDS; KC is a template argument so that the counting loop has no branch.
constexpr int kPerLane = (kFilterMax + 63) / 64;
template <int KC>
__device__ void rank_wave(const float* v, int n, int lane, float* srt, int16_t* ord) {
  float xs[KC];
  int rs[KC];
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int i = lane + 64 * k;
    xs[k] = i < n ? v[i] : 0.0f;
    rs[k] = 0;
  }
  for (int j = 0; j < n; ++j) {
    const float y = v[j];
#pragma unroll
    for (int k = 0; k < KC; ++k)  // branch-free: bitwise, not short-circuit, operators
      rs[k] += (int)(y < xs[k]) | ((int)(y == xs[k]) & (int)(j < lane + 64 * k));
  }
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int i = lane + 64 * k;
    if (i < n) {
      srt[rs[k]] = xs[k];
      ord[rs[k]] = (int16_t)i;
    }
  }
}

__global__ __launch_bounds__(64) void j2_filters_wave(const float* __restrict__ w, int n,
                                                      uint8_t* __restrict__ keep,
                                                      int* __restrict__ split,
                                                      double* __restrict__ gvf) {
  extern __shared__ float lds_f[];
  const int lane = threadIdx.x;
  const int64_t f = blockIdx.x;
  float* v = lds_f;
  float* srt = v + n;
  int16_t* ord = reinterpret_cast<int16_t*>(srt + n);
  for (int i = lane; i < n; i += 64) v[i] = w[f * n + i];
  __syncthreads();
  const int kc = (n + 63) / 64;
  if (kc <= 1)
    rank_wave<1>(v, n, lane, srt, ord);
  else if (kc <= 2)
    rank_wave<2>(v, n, lane, srt, ord);
  else if (kc <= 4)
    rank_wave<4>(v, n, lane, srt, ord);
  else if (kc <= 8)
    rank_wave<8>(v, n, lane, srt, ord);
  else
    rank_wave<kPerLane>(v, n, lane, srt, ord);
  __syncthreads();
  double* P = reinterpret_cast<double*>(reinterpret_cast<uint8_t*>(lds_f) + wave_sums_offset(n));
  double* Q = P + n;
  double* tot = Q + n;
  if (lane == 0) filter_prefix(srt, n, P, Q, tot);
  __syncthreads();
  const double pt = tot[0], qt = tot[1];
  double best = 0.0, ssd0 = 0.0;
  int arg = -1;
  for (int i = lane; i < n; i += 64) {  // ascending per lane: the lane's first minimum
    const double p = P[i], q = Q[i];
    const double left = i == 0 ? 0.0 : q - (p * p) / (double)i;
    const double rp = pt - p;
    const double right = (qt - q) - (rp * rp) / (double)(n - i);
    const double val = left + right;
    if (arg < 0 || val < best) {
      best = val;
      arg = i;
    }
    if (i == 0) ssd0 = val;
  }
  for (int m = 32; m >= 1; m >>= 1) {  // the smallest (value, index), lanes without one last
    const double ob = __shfl_xor(best, m, 64);
    const int oa = __shfl_xor(arg, m, 64);
    if (oa >= 0 && (arg < 0 || ob < best || (ob == best && oa < arg))) {
      best = ob;
      arg = oa;
    }
  }
  if (lane == 0) {
    split[f] = arg;
    gvf[f] = (ssd0 - best) / (ssd0 + 1e-8);
  }
  for (int r = lane; r < n; r += 64) keep[f * n + ord[r]] = r >= arg ? 1 : 0;
}

// ---------------------------------------------------------------------------------
// The per-split SSD of arrays that arrive sorted: the reference's jenks_optimization_cuda /
// jenks_optimization_biases_cuda (cuda_helpers.py:151-211, :85-146) and, per filter,
// jenks_optimization_cuda_conv (:219-289), which return var[idx] for every split and leave
// the argmin to the caller (JenksSGD and the other optimizers, custom_optimizer.py:135-136,
// :164-165).  The same sums as the mask path (no sort: the values are taken in the order
// given), the SSD of each split rounded to the input's type.
// ---------------------------------------------------------------------------------
// Workspace of the whole-array version: the block / superblock sums of j2_block_totals,
// j2_super, j2_top and j2_ssd (no sort buffers).
struct J2SsdLayout {
  int64_t nblk, nsup;
  size_t off_t1, off_t2, off_bx1, off_bx2, off_u1, off_u2, off_sx1, off_sx2;
  size_t off_bmin, off_bidx, off_ssd0, total;
};

J2SsdLayout j2_ssd_layout(int64_t n) {
  J2SsdLayout L;
  L.nblk = (n + kBlk - 1) / kBlk;
  L.nsup = (L.nblk + kSup - 1) / kSup;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o = align256(o + bytes);
    return at;
  };
  L.off_t1 = take(8 * (size_t)L.nblk);
  L.off_t2 = take(8 * (size_t)L.nblk);
  L.off_bx1 = take(8 * (size_t)L.nblk);
  L.off_bx2 = take(8 * (size_t)L.nblk);
  L.off_u1 = take(8 * (size_t)L.nsup);
  L.off_u2 = take(8 * (size_t)L.nsup);
  L.off_sx1 = take(8 * (size_t)(L.nsup + 1));
  L.off_sx2 = take(8 * (size_t)(L.nsup + 1));
  L.off_bmin = take(8 * (size_t)L.nblk);
  L.off_bidx = take(4 * (size_t)L.nblk);
  L.off_ssd0 = take(8);
  L.total = o;
  return L;
}

template <typename T>
int ssd_gpu(const T* srt, int64_t n, T* out, void* ws, hipStream_t hs) {
  const J2SsdLayout L = j2_ssd_layout(n);
  uint8_t* base = static_cast<uint8_t*>(ws);
  auto at = [&](size_t off) { return reinterpret_cast<double*>(base + off); };
  const int ni = (int)n, nblk = (int)L.nblk, nsup = (int)L.nsup;
  hipLaunchKernelGGL(j2_block_totals<T>, dim3(grid_of(nblk, 64)), dim3(64), 0, hs, srt, ni, nblk,
                     at(L.off_t1), at(L.off_t2));
  hipLaunchKernelGGL(j2_super, dim3(grid_of(nsup, 64)), dim3(64), 0, hs, at(L.off_t1),
                     at(L.off_t2), nblk, nsup, at(L.off_bx1), at(L.off_bx2), at(L.off_u1),
                     at(L.off_u2));
  hipLaunchKernelGGL(j2_top, dim3(1), dim3(kTopThreads), 0, hs, at(L.off_u1), at(L.off_u2), nsup,
                     at(L.off_sx1), at(L.off_sx2));
  hipLaunchKernelGGL(j2_ssd<T>, dim3(grid_of(nblk, 64)), dim3(64), 0, hs, srt, ni, nblk, nsup,
                     at(L.off_bx1), at(L.off_bx2), at(L.off_sx1), at(L.off_sx2), at(L.off_bmin),
                     reinterpret_cast<int*>(base + L.off_bidx), at(L.off_ssd0), out);
  return hipGetLastError() == hipSuccess ? FB_OK : FB_ERR_HIP;
}

// Every split's SSD of one sorted filter (n <= kFilterMax values: one superblock of at most
// four blocks), in the host's association order (every addition it makes, zeros included).
template <typename T>
__device__ void filter_ssd(const T* __restrict__ srt, int n, T* __restrict__ out) {
  const int nblk = (n + kBlk - 1) / kBlk;
  const double c = (double)srt[n / 2];
  double t1[4], t2[4], bx1[4], bx2[4];
  for (int b = 0; b < nblk; ++b) {
    double a1 = 0.0, a2 = 0.0;
    for (int i = b * kBlk; i < min(n, b * kBlk + kBlk); ++i) {
      const double d = (double)srt[i] - c;
      const double q = d * d;
      a1 = a1 + d;
      a2 = a2 + q;
    }
    t1[b] = a1;
    t2[b] = a2;
  }
  double u1, u2;
  {
    double a1 = 0.0, a2 = 0.0;
    for (int b = 0; b < nblk; ++b) {
      bx1[b] = a1;
      bx2[b] = a2;
      a1 = a1 + t1[b];
      a2 = a2 + t2[b];
    }
    u1 = a1;
    u2 = a2;
  }
  const double sx1 = 0.0, sx2 = 0.0;
  const double pt = 0.0 + u1, qt = 0.0 + u2;
  for (int b = 0; b < nblk; ++b) {
    const double base1 = sx1 + bx1[b], base2 = sx2 + bx2[b];
    double l1 = 0.0, l2 = 0.0;
    for (int i = b * kBlk; i < min(n, b * kBlk + kBlk); ++i) {
      const double p = base1 + l1, q = base2 + l2;
      const double left = i == 0 ? 0.0 : q - (p * p) / (double)i;
      const double rp = pt - p;
      const double right = (qt - q) - (rp * rp) / (double)(n - i);
      out[i] = (T)(left + right);
      const double d = (double)srt[i] - c;
      const double dq = d * d;
      l1 = l1 + d;
      l2 = l2 + dq;
    }
  }
}

// One thread per filter (as the reference's conv kernel runs one per (in, out) pair).
template <typename T>
__global__ __launch_bounds__(256) void j2_ssd_filters(const T* __restrict__ srt, int64_t nf,
                                                      int n, T* __restrict__ out) {
  const int64_t f = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (f < nf) filter_ssd(srt + f * n, n, out + f * n);
}

}  // namespace

extern "C" {

int fb_jenks2_ssd_workspace(int64_t n, size_t* bytes) {
  if (!bytes) return FB_ERR_NULL;
  if (n < 1 || n > INT32_MAX) return FB_ERR_SHAPE;
  *bytes = j2_ssd_layout(n).total;
  return FB_OK;
}

int fb_jenks2_ssd_gpu(const void* sorted, int64_t n, int32_t dtype, void* ssd, void* ws,
                      size_t ws_bytes, void* stream) {
  if (!sorted || !ssd || !ws) return FB_ERR_NULL;
  if (n < 1 || n > INT32_MAX) return FB_ERR_SHAPE;
  if (dtype != FB_DT_F32 && dtype != FB_DT_F64) return FB_ERR_DTYPE;
  if ((reinterpret_cast<uintptr_t>(sorted) & 15u) || (reinterpret_cast<uintptr_t>(ssd) & 15u) ||
      (reinterpret_cast<uintptr_t>(ws) & 255u))
    return FB_ERR_ALIGN;
  if (ws_bytes < j2_ssd_layout(n).total) return FB_ERR_WORKSPACE;
  hipStream_t hs = static_cast<hipStream_t>(stream);
  if (dtype == FB_DT_F32)
    return ssd_gpu(static_cast<const float*>(sorted), n, static_cast<float*>(ssd), ws, hs);
  return ssd_gpu(static_cast<const double*>(sorted), n, static_cast<double*>(ssd), ws, hs);
}

int fb_jenks2_ssd_filters_gpu(const void* sorted, int64_t nf, int32_t n, int32_t dtype, void* ssd,
                              void* stream) {
  if (!sorted || !ssd) return FB_ERR_NULL;
  if (nf < 1 || n < 1 || n > FB_JENKS2_FILTER_MAX || nf > INT32_MAX) return FB_ERR_SHAPE;
  if (dtype != FB_DT_F32 && dtype != FB_DT_F64) return FB_ERR_DTYPE;
  const uintptr_t a = dtype == FB_DT_F32 ? 3u : 7u;
  if ((reinterpret_cast<uintptr_t>(sorted) & a) || (reinterpret_cast<uintptr_t>(ssd) & a))
    return FB_ERR_ALIGN;
  hipStream_t hs = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((nf + 255) / 256));
  if (dtype == FB_DT_F32)
    hipLaunchKernelGGL(j2_ssd_filters<float>, grid, dim3(256), 0, hs,
                       static_cast<const float*>(sorted), nf, (int)n, static_cast<float*>(ssd));
  else
    hipLaunchKernelGGL(j2_ssd_filters<double>, grid, dim3(256), 0, hs,
                       static_cast<const double*>(sorted), nf, (int)n, static_cast<double*>(ssd));
  return hipGetLastError() == hipSuccess ? FB_OK : FB_ERR_HIP;
}

int fb_jenks2_workspace(int64_t n, size_t* bytes) {
  if (!bytes) return FB_ERR_NULL;
  if (n < 1 || n > INT32_MAX) return FB_ERR_SHAPE;
  J2Layout L;
  const int st = j2_layout(n, L);
  if (st != FB_OK) return st;
  *bytes = L.total;
  return FB_OK;
}

int fb_jenks2_gpu(const float* w, int64_t n, uint8_t* keep, int64_t* split, double* gvf,
                  void* ws, size_t ws_bytes, void* stream) {
  if (!w || !keep || !split || !gvf || !ws) return FB_ERR_NULL;
  if (n < 1 || n > INT32_MAX) return FB_ERR_SHAPE;
  if ((reinterpret_cast<uintptr_t>(ws) & 255u) || (reinterpret_cast<uintptr_t>(split) & 7u) ||
      (reinterpret_cast<uintptr_t>(gvf) & 7u) || (reinterpret_cast<uintptr_t>(w) & 3u))
    return FB_ERR_ALIGN;
  J2Layout L;
  int st = j2_layout(n, L);
  if (st != FB_OK) return st;
  if (ws_bytes < L.total) return FB_ERR_WORKSPACE;
  hipStream_t hs = static_cast<hipStream_t>(stream);
  uint8_t* base = static_cast<uint8_t*>(ws);
  auto at = [&](size_t off) { return static_cast<void*>(base + off); };
  float* keys_in = static_cast<float*>(at(L.off_keys_in));
  float* keys_out = static_cast<float*>(at(L.off_keys_out));
  int* vals_in = static_cast<int*>(at(L.off_vals_in));
  int* vals_out = static_cast<int*>(at(L.off_vals_out));
  double *t1 = static_cast<double*>(at(L.off_t1)), *t2 = static_cast<double*>(at(L.off_t2));
  double *bx1 = static_cast<double*>(at(L.off_bx1)), *bx2 = static_cast<double*>(at(L.off_bx2));
  double *u1 = static_cast<double*>(at(L.off_u1)), *u2 = static_cast<double*>(at(L.off_u2));
  double *sx1 = static_cast<double*>(at(L.off_sx1)), *sx2 = static_cast<double*>(at(L.off_sx2));
  double* bmin = static_cast<double*>(at(L.off_bmin));
  int* bidx = static_cast<int*>(at(L.off_bidx));
  double* smin = static_cast<double*>(at(L.off_smin));
  int* sidx = static_cast<int*>(at(L.off_sidx));
  double* ssd0 = static_cast<double*>(at(L.off_ssd0));
  const int ni = (int)n, nblk = (int)L.nblk, nsup = (int)L.nsup;
  hipLaunchKernelGGL(j2_prep, dim3(grid_of(n, 256)), dim3(256), 0, hs, w, keys_in, vals_in, ni);
  size_t sb = L.sort_bytes;
  if (hipcub::DeviceRadixSort::SortPairs(at(L.off_sort), sb, keys_in, keys_out, vals_in, vals_out,
                                         ni, 0, 32, hs) != hipSuccess)
    return FB_ERR_HIP;
  hipLaunchKernelGGL(j2_block_totals<float>, dim3(grid_of(nblk, 64)), dim3(64), 0, hs, keys_out, ni,
                     nblk, t1, t2);
  hipLaunchKernelGGL(j2_super, dim3(grid_of(nsup, 64)), dim3(64), 0, hs, t1, t2, nblk, nsup, bx1,
                     bx2, u1, u2);
  hipLaunchKernelGGL(j2_top, dim3(1), dim3(kTopThreads), 0, hs, u1, u2, nsup, sx1, sx2);
  hipLaunchKernelGGL(j2_ssd<float>, dim3(grid_of(nblk, 64)), dim3(64), 0, hs, keys_out, ni, nblk,
                     nsup, bx1, bx2, sx1, sx2, bmin, bidx, ssd0, (float*)nullptr);
  hipLaunchKernelGGL(j2_min_super, dim3(nsup), dim3(64), 0, hs, bmin, bidx, nblk, nsup, smin,
                     sidx);
  hipLaunchKernelGGL(j2_final, dim3(1), dim3(kFinalThreads), 0, hs, smin, sidx, nsup, ssd0, split,
                     gvf);
  hipLaunchKernelGGL(j2_mask, dim3(grid_of(n, 256)), dim3(256), 0, hs, w, keys_out, vals_out, ni,
                     split, keep);
  return hipGetLastError() == hipSuccess ? FB_OK : FB_ERR_HIP;
}

int fb_jenks2_filters_gpu(const float* w, int64_t nf, int32_t n, uint8_t* keep, int32_t* split,
                          double* gvf, void* stream) {
  if (!w || !keep || !split || !gvf) return FB_ERR_NULL;
  if (nf < 1 || n < 1 || n > FB_JENKS2_FILTER_MAX || nf > INT32_MAX) return FB_ERR_SHAPE;
  if ((reinterpret_cast<uintptr_t>(w) & 3u) || (reinterpret_cast<uintptr_t>(split) & 3u) ||
      (reinterpret_cast<uintptr_t>(gvf) & 7u))
    return FB_ERR_ALIGN;
  hipStream_t hs = static_cast<hipStream_t>(stream);
  if (n <= kLaneFilterMax && nf >= kLaneFilterMin)
    hipLaunchKernelGGL(j2_filters_lane, dim3((unsigned)((nf + 255) / 256)), dim3(256),
                       (size_t)256 * n * 10, hs, w, nf, (int)n, keep, split, gvf);
  else
    hipLaunchKernelGGL(j2_filters_wave, dim3((unsigned)nf), dim3(64),
                       wave_lds_bytes(n), hs, w, (int)n, keep, split, gvf);
  return hipGetLastError() == hipSuccess ? FB_OK : FB_ERR_HIP;
}

}  // extern "C"
