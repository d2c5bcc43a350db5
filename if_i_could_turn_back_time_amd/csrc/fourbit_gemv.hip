// Fused 4-bit dequant-GEMV for gfx950 (MI355X), batch 1..4, and the device decoder.
//
// One workgroup = 8 wave64s.  Each workgroup stages the activation x[B,K] in LDS
// (optionally rotating it with a blockwise FWHT first), then every wave streams a
// contiguous range of whole rows of the weight.  The weight is cut into items of 128
// K-elements of one row (see fourbit_layout.h); lane l of a wave takes item
// i0 + l + 64*s at step s, so each global_load_dwordx4 of the wave reads 1 KiB of
// consecutive bytes.  A lane decodes its item in registers (GF4: two v_perm_b32
// lookups per byte plane merged by XOR; E2M1: v_cvt_scalef32_pk_{bf16,f16}_fp4),
// multiplies with v_dot2_f32_{f16,bf16} into fp32 partials, and the wave folds the
// partials of each row with a DPP reduction.  Rows never straddle waves, so every
// output is written once and results do not depend on scheduling.
#include <hip/hip_runtime.h>

#include <atomic>

#include "fourbit.h"
#include "fourbit_layout.h"

namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf162_t __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kLdsLimit = 160 * 1024;

// ---------------------------------------------------------------------------------
// small device helpers
// ---------------------------------------------------------------------------------
__device__ __forceinline__ unsigned perm(unsigned s0, unsigned s1, unsigned sel) {
  return __builtin_amdgcn_perm(s0, s1, sel);
}

__device__ __forceinline__ float dot2_f16(unsigned w, unsigned x, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, w), __builtin_bit_cast(half2_t, x),
                                acc, false);
}

__device__ __forceinline__ float dot2_bf16(unsigned w, unsigned x, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf162_t, w),
                                         __builtin_bit_cast(bf162_t, x), acc, false);
}

template <int CTRL, int ROWMASK>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWMASK, 0xF, false));
}

// Sum over the 64 lanes; the result is returned uniformly.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141, 0xF>(v);  // row_half_mirror
  v += dpp_f<0x140, 0xF>(v);  // row_mirror
  v += dpp_f<0x142, 0xA>(v);  // row_bcast:15 into rows 1, 3
  v += dpp_f<0x143, 0xC>(v);  // row_bcast:31 into rows 2, 3
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
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

// ---------------------------------------------------------------------------------
// GF4 decode of one 32-bit word (8 codes, layout order) into 4 fp16 pairs in
// element order (e0,e1) (e2,e3) (e4,e5) (e6,e7).
// tl/th: lo/hi byte-plane tables {A'[0..3], A'[4..7], B'[0..3], B'[4..7]}.
// ---------------------------------------------------------------------------------
__device__ __forceinline__ void gf4_decode8(unsigned q, const u32x4& tl, const u32x4& th,
                                            unsigned w[4]) {
  const unsigned sa = q & 0x0F0F0F0Fu;
  const unsigned sb = (q >> 4) & 0x0F0F0F0Fu;
  const unsigned sa8 = sa ^ 0x08080808u;
  const unsigned sb8 = sb ^ 0x08080808u;
  const unsigned loA = perm(tl.y, tl.x, sa) ^ perm(tl.w, tl.z, sa8);
  const unsigned hiA = perm(th.y, th.x, sa) ^ perm(th.w, th.z, sa8);
  const unsigned loB = perm(tl.y, tl.x, sb) ^ perm(tl.w, tl.z, sb8);
  const unsigned hiB = perm(th.y, th.x, sb) ^ perm(th.w, th.z, sb8);
  w[0] = perm(hiA, loA, 0x05010400u);
  w[1] = perm(hiA, loA, 0x07030602u);
  w[2] = perm(hiB, loB, 0x05010400u);
  w[3] = perm(hiB, loB, 0x07030602u);
}

// E2M1 decode of byte j of q (elements 2j, 2j+1) into a 16-bit pair, unscaled.
template <int XDT, int J>
__device__ __forceinline__ unsigned e2m1_decode2(unsigned q) {
  if constexpr (XDT == FB_DT_BF16) {
    return __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, 1.0f, J));
  } else {
    return __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q, 1.0f, J));
  }
}

// ---------------------------------------------------------------------------------
// Per-item records
// ---------------------------------------------------------------------------------
template <int FMT>
struct Rec {
  u32x4 nib[4];
  u32x4 t0, t1;  // GF4: lo / hi tables.  E2M1: t0.x holds the 4 scale bytes.
};

template <int FMT>
__device__ __forceinline__ void load_rec(const uint8_t* __restrict__ w, int item, Rec<FMT>& r) {
  constexpr int BB = FMT == FB_FMT_GF4 ? fb::kGf4BlockBytes : fb::kE2m1BlockBytes;
  const uint8_t* base = w + (int64_t)(item >> 6) * BB + (item & 63) * 16;
#pragma unroll
  for (int c = 0; c < 4; ++c) r.nib[c] = ldg16(base + c * 1024);
  if constexpr (FMT == FB_FMT_GF4) {
    r.t0 = ldg16(base + 4096);
    r.t1 = ldg16(base + 5120);
  } else {
    const uint8_t* sp = w + (int64_t)(item >> 6) * BB + 4096 + (item & 63) * 4;
    r.t0.x = __builtin_nontemporal_load(reinterpret_cast<const unsigned*>(sp));
  }
}

// Partial dot products of one item with the staged activation slice.
// xs: LDS slice base (batch b at xs + b*256 bytes, 128 x 16-bit values each).
template <int FMT, int B, int XDT>
__device__ __forceinline__ void item_dot(const Rec<FMT>& r, const uint8_t* xs, float acc[B]) {
  if constexpr (FMT == FB_FMT_GF4) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        unsigned w[4];
        gf4_decode8(r.nib[c][d], r.t0, r.t1, w);
#pragma unroll
        for (int b = 0; b < B; ++b) {
          const u32x4 xv = *reinterpret_cast<const u32x4*>(xs + b * 256 + (c * 32 + d * 8) * 2);
          acc[b] = dot2_f16(w[0], xv.x, acc[b]);
          acc[b] = dot2_f16(w[1], xv.y, acc[b]);
          acc[b] = dot2_f16(w[2], xv.z, acc[b]);
          acc[b] = dot2_f16(w[3], xv.w, acc[b]);
        }
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float part[B];
#pragma unroll
      for (int b = 0; b < B; ++b) part[b] = 0.0f;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const unsigned q = r.nib[c][d];
        const unsigned w0 = e2m1_decode2<XDT, 0>(q);
        const unsigned w1 = e2m1_decode2<XDT, 1>(q);
        const unsigned w2 = e2m1_decode2<XDT, 2>(q);
        const unsigned w3 = e2m1_decode2<XDT, 3>(q);
#pragma unroll
        for (int b = 0; b < B; ++b) {
          const u32x4 xv = *reinterpret_cast<const u32x4*>(xs + b * 256 + (c * 32 + d * 8) * 2);
          if constexpr (XDT == FB_DT_BF16) {
            part[b] = dot2_bf16(w0, xv.x, part[b]);
            part[b] = dot2_bf16(w1, xv.y, part[b]);
            part[b] = dot2_bf16(w2, xv.z, part[b]);
            part[b] = dot2_bf16(w3, xv.w, part[b]);
          } else {
            part[b] = dot2_f16(w0, xv.x, part[b]);
            part[b] = dot2_f16(w1, xv.y, part[b]);
            part[b] = dot2_f16(w2, xv.z, part[b]);
            part[b] = dot2_f16(w3, xv.w, part[b]);
          }
        }
      }
      const int e = (int)((r.t0.x >> (8 * c)) & 0xFFu) - 127;
#pragma unroll
      for (int b = 0; b < B; ++b) acc[b] += __builtin_ldexpf(part[b], e);
    }
  }
}

// ---------------------------------------------------------------------------------
// Activation staging.  Slice g (128 values) of batch row b lives at
// g*(B*256+16) + b*256 bytes: the 16-byte pad per slice spreads lanes that read
// neighbouring slices over all LDS banks.
// ---------------------------------------------------------------------------------
template <int B>
__device__ __forceinline__ void stage_plain(uint8_t* lds, const uint16_t* __restrict__ x, int K) {
  const int ss = B * 256 + 16;
  const int per_row = K >> 3;  // 16-byte chunks per batch row
  for (int t = threadIdx.x; t < B * per_row; t += kThreads) {
    const int b = t / per_row;
    const int k8 = (t - b * per_row) << 3;
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + (int64_t)b * K + k8);
    *reinterpret_cast<u32x4*>(lds + (k8 >> 7) * ss + b * 256 + (k8 & 127) * 2) = v;
  }
}

// Blockwise normalised FWHT of x (fp16) in fp32, result rounded to fp16 into the
// slices.  F (B*K floats) is LDS scratch.  Stages are done 4 at a time: a thread owns
// 16 values spaced h0 apart and applies strides h0, 2h0, 4h0, 8h0 in registers.
template <int B>
__device__ __forceinline__ void stage_fwht(uint8_t* lds, float* F, const _Float16* __restrict__ x,
                                           int K, int fb) {
  const int ss = B * 256 + 16;
  for (int t = threadIdx.x; t < B * K; t += kThreads) F[t] = (float)x[t];
  __syncthreads();
  const int lg_fb = 31 - __builtin_clz(fb);
  for (int lg_h0 = 0; lg_h0 < lg_fb; lg_h0 += 4) {
    const int lg_span = min(4, lg_fb - lg_h0);
    const int span = 1 << lg_span;
    const int h0 = 1 << lg_h0;
    const int lg_nhi = lg_fb - lg_h0 - lg_span;
    const int ngroups = (B * K) >> lg_span;
    for (int t = threadIdx.x; t < ngroups; t += kThreads) {
      const int lo = t & (h0 - 1);
      const int rest = t >> lg_h0;
      const int hi = rest & ((1 << lg_nhi) - 1);
      const int blk = rest >> lg_nhi;
      float* base = F + blk * fb + ((hi << lg_span) << lg_h0) + lo;
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = u < span ? base[u * h0] : 0.0f;
#pragma unroll
      for (int s = 1; s < 16; s <<= 1) {
        if (s < span) {
#pragma unroll
          for (int u = 0; u < 16; ++u) {
            if ((u & s) == 0) {
              const float a = v[u], c = v[u + s];
              v[u] = a + c;
              v[u + s] = a - c;
            }
          }
        }
      }
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (u < span) base[u * h0] = v[u];
    }
    __syncthreads();
  }
  const float sc = 1.0f / __builtin_sqrtf((float)fb);
  for (int t = threadIdx.x; t < B * K; t += kThreads) {
    const int b = t / K;
    const int k = t - b * K;
    *reinterpret_cast<_Float16*>(lds + (k >> 7) * ss + b * 256 + (k & 127) * 2) =
        (_Float16)(F[t] * sc);
  }
}

// ---------------------------------------------------------------------------------
// The GEMV kernel
// ---------------------------------------------------------------------------------
template <int FMT, int B, int XDT>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const uint8_t* __restrict__ w,
                                                        const void* __restrict__ x,
                                                        void* __restrict__ y, int N, int K,
                                                        int fwht_block, int rows_per_wave,
                                                        int ydt) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int ipr = K >> 7;
  const int ss = B * 256 + 16;
  if (fwht_block) {
    stage_fwht<B>(lds, reinterpret_cast<float*>(lds + ipr * ss),
                  static_cast<const _Float16*>(x), K, fwht_block);
  } else {
    stage_plain<B>(lds, static_cast<const uint16_t*>(x), K);
  }
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * kWaves + (threadIdx.x >> 6);
  const int r0 = wave * rows_per_wave;
  const int r1 = min(N, r0 + rows_per_wave);
  if (r0 >= r1) return;
  const int i_begin = r0 * ipr;
  const int i_end = r1 * ipr;

  // lane position (row, slice) of item i_begin + lane, advanced by 64 per step
  int row = r0 + lane / ipr;
  int slice = lane - (lane / ipr) * ipr;
  // wave position of the step's first item
  int rlo = r0;
  int sb_slice = 0;

  float carry[B];
#pragma unroll
  for (int b = 0; b < B; ++b) carry[b] = 0.0f;

  Rec<FMT> cur, nxt;
  int item = i_begin + lane;
  if (item < i_end) load_rec<FMT>(w, item, cur);

  for (int sb = i_begin; sb < i_end; sb += 64) {
    const int inext = item + 64;
    if (inext < i_end) load_rec<FMT>(w, inext, nxt);

    float p[B];
#pragma unroll
    for (int b = 0; b < B; ++b) p[b] = 0.0f;
    const bool valid = item < i_end;
    if (valid) item_dot<FMT, B, XDT>(cur, lds + slice * ss, p);

    // rows touched by this step: rlo .. rhi
    const int slast = min(sb + 63, i_end - 1);
    int rhi = rlo;
    int t = sb_slice + (slast - sb);
    while (t >= ipr) {
      t -= ipr;
      ++rhi;
    }
    for (int r = rlo; r <= rhi; ++r) {
      const bool mine = valid && row == r;
      const bool done = (r + 1) * ipr - 1 <= slast;
#pragma unroll
      for (int b = 0; b < B; ++b) {
        float tot = wave_sum(mine ? p[b] : 0.0f);
        if (r == rlo) {
          tot += carry[b];
          carry[b] = 0.0f;
        }
        if (done) {
          if (lane == 0) store_y(y, (int64_t)b * N + r, tot, ydt);
        } else {
          carry[b] = tot;
        }
      }
    }

    // advance
    item = inext;
    slice += 64;
    while (slice >= ipr) {
      slice -= ipr;
      ++row;
    }
    sb_slice += 64;
    while (sb_slice >= ipr) {
      sb_slice -= ipr;
      ++rlo;
    }
    cur = nxt;
  }
}

// ---------------------------------------------------------------------------------
// Device decode: one thread per item writes 128 values.
// ---------------------------------------------------------------------------------
template <int FMT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ w,
                                                      void* __restrict__ out, int N, int K,
                                                      int odt) {
  const int ipr = K >> 7;
  const int item = blockIdx.x * 256 + threadIdx.x;
  if (item >= N * ipr) return;
  const int n = item / ipr;
  const int g = item - n * ipr;
  Rec<FMT> r;
  load_rec<FMT>(w, item, r);
  const int64_t o0 = (int64_t)n * K + g * 128;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      unsigned pr[4];
      float scale_e = 0;
      int e = 0;
      if constexpr (FMT == FB_FMT_GF4) {
        gf4_decode8(r.nib[c][d], r.t0, r.t1, pr);
      } else {
        const unsigned q = r.nib[c][d];
        pr[0] = e2m1_decode2<FB_DT_BF16, 0>(q);
        pr[1] = e2m1_decode2<FB_DT_BF16, 1>(q);
        pr[2] = e2m1_decode2<FB_DT_BF16, 2>(q);
        pr[3] = e2m1_decode2<FB_DT_BF16, 3>(q);
        e = (int)((r.t0.x >> (8 * c)) & 0xFFu) - 127;
      }
      (void)scale_e;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const unsigned bits = (pr[j] >> (16 * h)) & 0xFFFFu;
          float v;
          if constexpr (FMT == FB_FMT_GF4) {
            v = (float)__builtin_bit_cast(_Float16, (unsigned short)bits);
          } else {
            v = __builtin_ldexpf(__builtin_bit_cast(float, bits << 16), e);
          }
          const int64_t o = o0 + c * 32 + d * 8 + j * 2 + h;
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
// host helpers
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

size_t gemv_lds_bytes(const fb_shape_t* s) {
  const size_t ipr = (size_t)s->K / 128;
  size_t b = ipr * (size_t)(s->B * 256 + 16);
  if (s->fwht_block) b += (size_t)s->B * s->K * 4;
  return b;
}

template <int FMT, int B, int XDT>
int launch_gemv(const void* wdev, const void* x, void* y, const fb_shape_t* s,
                hipStream_t stream) {
  auto kern = gemv_kernel<FMT, B, XDT>;
  const size_t lds = gemv_lds_bytes(s);
  static std::atomic<bool> attr_set{false};
  if (!attr_set.load(std::memory_order_acquire)) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kLdsLimit) != hipSuccess)
      return FB_ERR_HIP;
    attr_set.store(true, std::memory_order_release);
  }
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return FB_ERR_HIP;
  const int cus = cu_count(dev);
  const int wg_per_cu = lds <= (size_t)kLdsLimit / 2 ? 2 : 1;
  const int ipr = s->K / 128;
  const int total_waves = cus * wg_per_cu * kWaves;
  int rpw = (s->N + total_waves - 1) / total_waves;
  const int min_rows = (64 + ipr - 1) / ipr;
  if (rpw < min_rows) rpw = min_rows;
  const int waves = (s->N + rpw - 1) / rpw;
  const int grid = (waves + kWaves - 1) / kWaves;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), lds, stream,
                     static_cast<const uint8_t*>(wdev), x, y, s->N, s->K, s->fwht_block, rpw,
                     s->y_dtype);
  return hipGetLastError() == hipSuccess ? FB_OK : FB_ERR_HIP;
}

template <int FMT, int XDT>
int dispatch_batch(const void* wdev, const void* x, void* y, const fb_shape_t* s,
                   hipStream_t st) {
  switch (s->B) {
    case 1: return launch_gemv<FMT, 1, XDT>(wdev, x, y, s, st);
    case 2: return launch_gemv<FMT, 2, XDT>(wdev, x, y, s, st);
    case 3: return launch_gemv<FMT, 3, XDT>(wdev, x, y, s, st);
    case 4: return launch_gemv<FMT, 4, XDT>(wdev, x, y, s, st);
    default: return FB_ERR_BATCH;
  }
}

}  // namespace

extern "C" {

size_t fb_workspace_bytes(const fb_shape_t* s) {
  (void)s;
  return 0;
}

int fb_gemv(const void* wdev, const void* x, void* y, const fb_shape_t* s, void* ws,
            size_t ws_bytes, void* stream) {
  (void)ws;
  (void)ws_bytes;
  if (!s || !wdev || !x || !y) return FB_ERR_NULL;
  int st = fb_validate(s);
  if (st != FB_OK) return st;
  if (s->B < 1 || s->B > 4) return FB_ERR_BATCH;
  if (!aligned16(wdev) || !aligned16(x) || (reinterpret_cast<uintptr_t>(y) & 3u))
    return FB_ERR_ALIGN;
  if (s->fwht_block && s->x_dtype != FB_DT_F16) return FB_ERR_DTYPE;
  if (gemv_lds_bytes(s) > (size_t)kLdsLimit) return FB_ERR_LDS;
  hipStream_t hs = static_cast<hipStream_t>(stream);
  if (s->fmt == FB_FMT_GF4) return dispatch_batch<FB_FMT_GF4, FB_DT_F16>(wdev, x, y, s, hs);
  if (s->x_dtype == FB_DT_BF16) return dispatch_batch<FB_FMT_E2M1, FB_DT_BF16>(wdev, x, y, s, hs);
  return dispatch_batch<FB_FMT_E2M1, FB_DT_F16>(wdev, x, y, s, hs);
}

int fb_dequant(const void* wdev, void* w_out, int32_t out_dtype, const fb_shape_t* s,
               void* stream) {
  if (!s || !wdev || !w_out) return FB_ERR_NULL;
  int st = fb_validate(s);
  if (st != FB_OK) return st;
  if (out_dtype != FB_DT_F32 && out_dtype != FB_DT_F16 && out_dtype != FB_DT_BF16)
    return FB_ERR_DTYPE;
  if (!aligned16(wdev)) return FB_ERR_ALIGN;
  const int items = s->N * (s->K / 128);
  const int grid = (items + 255) / 256;
  hipStream_t hs = static_cast<hipStream_t>(stream);
  if (s->fmt == FB_FMT_GF4)
    hipLaunchKernelGGL(dequant_kernel<FB_FMT_GF4>, dim3(grid), dim3(256), 0, hs,
                       static_cast<const uint8_t*>(wdev), w_out, s->N, s->K, out_dtype);
  else
    hipLaunchKernelGGL(dequant_kernel<FB_FMT_E2M1>, dim3(grid), dim3(256), 0, hs,
                       static_cast<const uint8_t*>(wdev), w_out, s->N, s->K, out_dtype);
  return hipGetLastError() == hipSuccess ? FB_OK : FB_ERR_HIP;
}

}  // extern "C"
