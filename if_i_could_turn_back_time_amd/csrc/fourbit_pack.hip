// Packers on the GPU, producing the same bytes as the host packers of fourbit_host.cpp:
// GF4 (the Jenks-16 and masked Jenks quantizer, one wavefront per (row, 128-group), fp64)
// and E2M1 (32 lanes per 32-group).
//
// Every fp64 expression is the host's, evaluated in the host's order, and this file is
// compiled with -ffp-contract=off (no fused multiply-adds), so each operation rounds
// exactly as on the CPU.  IEEE fp64 add/mul/div are correctly rounded on gfx950 and the
// conversions fp64 -> fp32 -> fp16 round to nearest even, so the outputs are bit-identical
// to fb_quantize_gf4 / fb_quantize_gf4_masked (and to the CPU oracle).
//
// Per group (one wave, LDS region of its own):
//   1. load 128 fp32 values (2 per lane) and the keep flags; compact the kept values in
//      index order with ballots (m of them);
//   2. stable rank by (value, index): rank = #{u : v_u < v} + #{u < t : v_u == v};
//   3. sequential fp64 prefix sums S1, S2 (one running sum, as the host);
//   4. the DP D[c][j] = min_{i >= c-1} D[c-1][i] + SSD(i, j) over classes c = 2..k, lane L
//      owning j = L+1 and j = L+65; the i loop is uniform across the wave (broadcast LDS
//      reads) and ascends, and only a strictly smaller candidate replaces: ties keep the
//      smallest break, as on the host;
//   5. lane 0 walks the back pointers; lanes 0..k-1 form the centroids; the codes are
//      scattered back to index order, nibble-packed, and written with the codebook.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdint>

#include "fourbit.h"

namespace {

constexpr int kGroup = 128;
constexpr int kMaxClasses = 16;

struct PackLds {
  double vs[kGroup];              // kept values, sorted
  double S1[kGroup + 1];          // prefix sums of vs
  double S2[kGroup + 1];          // prefix sums of vs^2
  double D[2][kGroup + 1];        // DP rows, alternating
  float sub[kGroup];              // kept values in index order
  uint8_t pos[kGroup];            // original index of sub[t]
  uint8_t order[kGroup];          // original index of vs[p]
  uint8_t back[kMaxClasses + 1][kGroup + 1];
  uint8_t code[kGroup];           // final code by original index
  int bounds[kMaxClasses + 1];
  uint16_t cb[kMaxClasses];
};

__device__ __forceinline__ double ssd(const PackLds& L, int i, int j, double S1j, double S2j) {
  const double s = S1j - L.S1[i];
  const double q = S2j - L.S2[i];
  return q - (s * s) / (double)(j - i);
}

__global__ __launch_bounds__(64) void gf4_pack_kernel(const float* __restrict__ w,
                                                      const uint8_t* __restrict__ keep,
                                                      int K, int64_t groups,
                                                      uint8_t* __restrict__ codes,
                                                      uint16_t* __restrict__ book) {
  __shared__ PackLds L;
  const int lane = threadIdx.x;
  const int G = K / kGroup;
  for (int64_t it = blockIdx.x; it < groups; it += gridDim.x) {
    const int64_t n = it / G, g = it - n * G;
    const int64_t off = n * K + g * kGroup;

    // 1. load and compact the kept values (index order)
    const float v0 = w[off + lane], v1 = w[off + lane + 64];
    const bool k0 = keep ? keep[off + lane] != 0 : true;
    const bool k1 = keep ? keep[off + lane + 64] != 0 : true;
    const uint64_t b0 = __ballot(k0), b1 = __ballot(k1);
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const int c0 = __popcll(b0);
    const int m = c0 + __popcll(b1);
    const bool full = m == kGroup;
    const int k = full ? kMaxClasses : (m < kMaxClasses - 1 ? m : kMaxClasses - 1);
    if (k0) {
      const int t = __popcll(b0 & below);
      L.sub[t] = v0;
      L.pos[t] = (uint8_t)lane;
    }
    if (k1) {
      const int t = c0 + __popcll(b1 & below);
      L.sub[t] = v1;
      L.pos[t] = (uint8_t)(lane + 64);
    }
    __syncthreads();

    // 2. stable rank by (value, index) -- the host's std::stable_sort on (double)value
    for (int h = 0; h < 2; ++h) {
      const int t = lane + 64 * h;
      const float vt = t < m ? L.sub[t] : 0.0f;
      int rank = 0;
      for (int u = 0; u < m; ++u) {
        const float vu = L.sub[u];
        rank += (vu < vt) || (vu == vt && u < t);
      }
      if (t < m) {
        L.vs[rank] = (double)vt;
        L.order[rank] = L.pos[t];
      }
    }
    __syncthreads();

    // 3. sequential prefix sums (every lane runs the same chain; lane 0 stores it)
    {
      double a = 0.0, b = 0.0;
      if (lane == 0) {
        L.S1[0] = 0.0;
        L.S2[0] = 0.0;
      }
      for (int t = 0; t < m; ++t) {
        const double x = L.vs[t];
        a = a + x;
        b = b + x * x;
        if (lane == 0) {
          L.S1[t + 1] = a;
          L.S2[t + 1] = b;
        }
      }
    }
    __syncthreads();

    // 4. DP over classes; lane owns columns j0 = lane+1 and j1 = lane+65 (valid if <= m)
    const double inf = __builtin_huge_val();
    const int j0 = lane + 1, j1 = lane + 65;
    const bool ok0 = j0 <= m, ok1 = j1 <= m;
    const double S1j0 = ok0 ? L.S1[j0] : 0.0, S2j0 = ok0 ? L.S2[j0] : 0.0;
    const double S1j1 = ok1 ? L.S1[j1] : 0.0, S2j1 = ok1 ? L.S2[j1] : 0.0;
    if (k > 0) {
      // one class: [0, j)
      if (lane == 0) L.D[0][0] = inf;
      if (ok0) L.D[0][j0] = ssd(L, 0, j0, S1j0, S2j0);
      if (ok1) L.D[0][j1] = ssd(L, 0, j1, S1j1, S2j1);
    }
    __syncthreads();
    int cur = 0;
    for (int c = 2; c <= k; ++c) {
      const double* Dp = L.D[cur];
      double best0 = inf, best1 = inf;
      int bi0 = 0, bi1 = 0;
      const int ilo = c - 1;
      // columns j0 <= 64 only see i < 64; columns j1 see every i < m
      const int imid = m < 64 ? m : 64;
      for (int i = ilo; i < imid; ++i) {
        const double d = Dp[i];
        if (i < j0 && ok0) {
          const double cand = d + ssd(L, i, j0, S1j0, S2j0);
          if (cand < best0) {
            best0 = cand;
            bi0 = i;
          }
        }
        if (ok1) {
          const double cand = d + ssd(L, i, j1, S1j1, S2j1);
          if (cand < best1) {
            best1 = cand;
            bi1 = i;
          }
        }
      }
      for (int i = (ilo > 64 ? ilo : 64); i < m; ++i) {
        if (ok1 && i < j1) {
          const double cand = Dp[i] + ssd(L, i, j1, S1j1, S2j1);
          if (cand < best1) {
            best1 = cand;
            bi1 = i;
          }
        }
      }
      // a prefix [0, j) with j < c cannot hold c non-empty classes
      if (j0 < c) best0 = inf;
      if (j1 < c) best1 = inf;
      double* Dn = L.D[cur ^ 1];
      if (lane == 0) {
        Dn[0] = inf;
        L.back[c][0] = 0;
      }
      if (ok0) {
        Dn[j0] = best0;
        L.back[c][j0] = (uint8_t)bi0;
      }
      if (ok1) {
        Dn[j1] = best1;
        L.back[c][j1] = (uint8_t)bi1;
      }
      cur ^= 1;
      __syncthreads();
    }

    // 5. breaks, centroids, codes
    if (lane == 0) {
      L.bounds[0] = 0;
      L.bounds[k] = m;
      int j = m;
      for (int c = k; c >= 2; --c) {
        const int i = L.back[c][j];
        L.bounds[c - 1] = i;
        j = i;
      }
    }
    __syncthreads();
    if (lane < k) {
      const int lo = L.bounds[lane], hi = L.bounds[lane + 1];
      const double mean = (L.S1[hi] - L.S1[lo]) / (double)(hi - lo);
      L.cb[lane] = __half_as_ushort(__float2half_rn((float)mean));
    }
    __syncthreads();
    // the zero entry of a masked group goes after the strictly negative centroids
    int z = 0;
    if (!full)
      for (int t = 0; t < k; ++t) z += ((L.cb[t] & 0x8000u) && (L.cb[t] & 0x7fffu)) ? 1 : 0;
    for (int h = 0; h < 2; ++h) {
      const int p = lane + 64 * h;
      L.code[p] = (uint8_t)z;  // masked entries
    }
    __syncthreads();
    for (int h = 0; h < 2; ++h) {
      const int p = lane + 64 * h;
      if (p < m) {
        int cls = 0;
        for (int c = 1; c < k; ++c) cls += (L.bounds[c] <= p) ? 1 : 0;
        L.code[L.order[p]] = (uint8_t)(full ? cls : cls + (cls >= z ? 1 : 0));
      }
    }
    __syncthreads();
    codes[n * (K / 2) + g * 64 + lane] = (uint8_t)(L.code[2 * lane] | (L.code[2 * lane + 1] << 4));
    if (lane < kMaxClasses) {
      uint16_t e;
      if (full) {
        e = L.cb[lane];
      } else {
        const int t = lane < k ? lane : k;  // entries past the last used one repeat it
        e = t < z ? L.cb[t] : (t == z ? (uint16_t)0 : L.cb[t - 1]);
      }
      book[it * kMaxClasses + lane] = e;
    }
    __syncthreads();
  }
}

// E2M1 + E8M0 per 32-group, 32 lanes per group (a wave packs two groups): the host
// packer's rule (fb_quantize_e2m1) in fp32, which is exact here: amax's exponent comes from
// frexp, q = v * 2^-e is a power-of-two scaling, and the rounding midpoints are fp32 values.
__device__ __forceinline__ int e2m1_index(float a) {
  const float mids[7] = {0.25f, 0.75f, 1.25f, 1.75f, 2.5f, 3.5f, 5.0f};
  int idx = 0;
  bool tie = false;
#pragma unroll
  for (int t = 0; t < 7; ++t) {
    idx += a > mids[t] ? 1 : 0;
    tie = tie || a == mids[t];
  }
  if (tie && (idx & 1)) ++idx;
  return idx < 7 ? idx : 7;
}

__global__ __launch_bounds__(256) void e2m1_pack_kernel(const float* __restrict__ w,
                                                        int64_t groups,
                                                        uint8_t* __restrict__ codes,
                                                        uint8_t* __restrict__ scales) {
  const int lane = threadIdx.x & 63;
  const int t = lane & 31;                        // value index in the group
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t it0 = wave * 2; it0 < groups; it0 += nwaves * 2) {  // uniform per wave
    const int64_t it = it0 + (lane >> 5);
    const bool live = it < groups;
    const float v = live ? w[it * 32 + t] : 0.0f;
    float amax = __builtin_fabsf(v);
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 32));
    int ex = 0;
    if (amax > 0.0f) {
      int e2;
      (void)frexpf(amax, &e2);  // amax = m * 2^e2, m in [0.5, 1)
      ex = e2 - 1 - 2;
      ex = ex < -127 ? -127 : (ex > 127 ? 127 : ex);
    }
    const float q = ldexpf(v, -ex);
    const int code = (__builtin_signbit(v) ? 8 : 0) | e2m1_index(__builtin_fabsf(q));
    const int hi = __shfl_xor(code, 1, 32);
    if (live && !(t & 1)) codes[it * 16 + (t >> 1)] = (uint8_t)(code | (hi << 4));
    if (live && t == 0) scales[it] = (uint8_t)(ex + 127);
  }
}

}  // namespace

extern "C" {

int fb_quantize_gf4_gpu(const float* w, const uint8_t* keep, int32_t N, int32_t K,
                        uint8_t* codes, uint16_t* codebook, void* stream) {
  if (!w || !codes || !codebook) return FB_ERR_NULL;
  if (N < 1 || K < 128 || K % 128) return FB_ERR_SHAPE;
  const int64_t groups = (int64_t)N * (K / kGroup);
  const int grid = (int)(groups < (1 << 22) ? groups : (1 << 22));
  hipLaunchKernelGGL(gf4_pack_kernel, dim3(grid), dim3(64), 0,
                     static_cast<hipStream_t>(stream), w, keep, K, groups, codes, codebook);
  return hipGetLastError() == hipSuccess ? FB_OK : FB_ERR_HIP;
}

}  // extern "C"

extern "C" int fb_quantize_e2m1_gpu(const float* w, int32_t N, int32_t K, uint8_t* codes,
                                    uint8_t* scales, void* stream) {
  if (!w || !codes || !scales) return FB_ERR_NULL;
  if (N < 1 || K < 128 || K % 128) return FB_ERR_SHAPE;
  const int64_t groups = (int64_t)N * (K / 32);
  const int64_t blocks = (groups + 7) / 8;  // 8 groups per 256-thread block
  const int grid = (int)(blocks < (1 << 20) ? blocks : (1 << 20));
  hipLaunchKernelGGL(e2m1_pack_kernel, dim3(grid), dim3(256), 0,
                     static_cast<hipStream_t>(stream), w, groups, codes, scales);
  return hipGetLastError() == hipSuccess ? FB_OK : FB_ERR_HIP;
}
