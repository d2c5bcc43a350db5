// Host side of libfourbit.so: argument validation, deterministic packers (GF4 Jenks-16,
// E2M1/E8M0), the offline FWHT weight rotation and the canonical <-> device weight
// stream transform.  Built with -ffp-contract=off so every fp64 expression rounds
// exactly as written (the packers must be bit-identical run to run and machine to
// machine).
#include "fourbit.h"
#include "fourbit_layout.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <limits>
#include <numeric>
#include <thread>
#include <vector>

namespace {

// ---------------------------------------------------------------------------------
// fp32 -> fp16 (IEEE binary16) round-to-nearest-even, including subnormals.
// ---------------------------------------------------------------------------------
uint16_t f32_to_f16_rne(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to >= 65520 -> inf
  if (ax < 0x38800000u) {                                    // |f| < 2^-14: subnormal half
    // value = ax_float; half subnormal unit = 2^-24
    const int e = (int)(ax >> 23);                           // biased fp32 exponent
    if (e < 102) return (uint16_t)sign;                      // < 2^-25: rounds to 0
    uint32_t mant = (ax & 0x7fffffu) | 0x800000u;            // 24-bit significand
    const int shift = 126 - e;                               // to units of 2^-24
    uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
  }
  uint32_t h = ((ax >> 13) - (112u << 10));  // rebias 127 -> 15
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  return (uint16_t)(sign | h);
}

float f16_bits_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 31u, m = h & 1023u;
  float v;
  if (e == 0) {
    v = std::ldexp((float)m, -24);  // subnormal (or zero)
  } else if (e == 31) {
    v = m ? std::numeric_limits<float>::quiet_NaN() : std::numeric_limits<float>::infinity();
  } else {
    v = std::ldexp((float)(1024u + m), (int)e - 25);
  }
  uint32_t bits;
  std::memcpy(&bits, &v, 4);
  bits |= sign;
  std::memcpy(&v, &bits, 4);
  return v;
}

// Runs fn(begin, end) over [0, n) split across up to nthreads std::threads.
template <class Fn>
void parallel_for(int64_t n, int nthreads, Fn fn) {
  if (n <= 0) return;
  int nt = (int)std::min<int64_t>(std::max(1, nthreads), n);
  if (nt == 1) {
    fn((int64_t)0, n);
    return;
  }
  std::vector<std::thread> th;
  th.reserve(nt);
  const int64_t chunk = (n + nt - 1) / nt;
  for (int t = 0; t < nt; ++t) {
    const int64_t b = t * chunk, e = std::min(n, b + chunk);
    if (b >= e) break;
    th.emplace_back([=] { fn(b, e); });
  }
  for (auto& x : th) x.join();
}

// ---------------------------------------------------------------------------------
// GF4: Jenks natural breaks with 16 classes on one group of n values.
// ---------------------------------------------------------------------------------
struct JenksScratch {
  std::vector<int> order;
  std::vector<double> v, S1, S2, ssd, Dp, Dc;
  std::vector<int> back;  // [k+1][n+1]
  explicit JenksScratch(int n, int k)
      : order(n), v(n), S1(n + 1), S2(n + 1), ssd((size_t)(n + 1) * (n + 1)), Dp(n + 1),
        Dc(n + 1), back((size_t)(k + 1) * (n + 1)) {}
};

// Quantizes one group: vals[n] -> codes[n] (class index) and book[k] (fp16 bits).
// Same arithmetic as the fp64 DP of the CPU oracle: sequential prefix sums,
// SSD(i,j) = (S2[j]-S2[i]) - (S1[j]-S1[i])^2/(j-i), D[m][j] = min_i D[m-1][i] + SSD(i,j)
// with the smallest i kept on ties (i ascends; only a strictly smaller candidate
// replaces), centroid (S1[hi]-S1[lo])/(hi-lo) rounded fp64 -> fp32 -> fp16.
void jenks_group(const float* vals, int n, int k, uint8_t* codes, uint16_t* book,
                 JenksScratch& S) {
  for (int t = 0; t < n; ++t) S.order[t] = t;
  std::stable_sort(S.order.begin(), S.order.begin() + n,
                   [&](int a, int b) { return (double)vals[a] < (double)vals[b]; });
  for (int t = 0; t < n; ++t) S.v[t] = (double)vals[S.order[t]];
  S.S1[0] = 0.0;
  S.S2[0] = 0.0;
  for (int t = 0; t < n; ++t) {
    S.S1[t + 1] = S.S1[t] + S.v[t];
    S.S2[t + 1] = S.S2[t] + S.v[t] * S.v[t];
  }
  const int W = n + 1;
  const double inf = std::numeric_limits<double>::infinity();
  for (int i = 0; i <= n; ++i) {
    double* row = &S.ssd[(size_t)i * W];
    for (int j = 0; j <= i; ++j) row[j] = inf;
    for (int j = i + 1; j <= n; ++j) {
      const double s = S.S1[j] - S.S1[i];
      const double q = S.S2[j] - S.S2[i];
      row[j] = q - (s * s) / (double)(j - i);
    }
  }
  // one class: [0, j)
  for (int j = 0; j <= n; ++j) S.Dp[j] = S.ssd[j];
  for (int m = 2; m <= k; ++m) {
    int* bk = &S.back[(size_t)m * W];
    for (int j = 0; j <= n; ++j) {
      S.Dc[j] = inf;
      bk[j] = 0;
    }
    for (int i = m - 1; i < n; ++i) {
      const double d = S.Dp[i];
      const double* row = &S.ssd[(size_t)i * W];
      for (int j = i + 1; j <= n; ++j) {
        const double c = d + row[j];
        const bool better = c < S.Dc[j];
        S.Dc[j] = better ? c : S.Dc[j];
        bk[j] = better ? i : bk[j];
      }
    }
    for (int j = 0; j < m; ++j) S.Dc[j] = inf;
    std::swap(S.Dp, S.Dc);
  }
  int bounds[17];
  bounds[0] = 0;
  bounds[k] = n;
  int j = n;
  for (int m = k; m >= 2; --m) {
    const int i = S.back[(size_t)m * W + j];
    bounds[m - 1] = i;
    j = i;
  }
  for (int c = 0; c < k; ++c) {
    const int lo = bounds[c], hi = bounds[c + 1];
    const double mean = (S.S1[hi] - S.S1[lo]) / (double)(hi - lo);
    book[c] = f32_to_f16_rne((float)mean);
    for (int p = lo; p < hi; ++p) codes[S.order[p]] = (uint8_t)c;
  }
}

// One group with a keep mask.  Masked entries take an exact-zero codebook entry; the
// kept values are partitioned into min(15, kept) classes by jenks_group.  The zero entry
// goes after every strictly negative centroid, so the codebook stays non-decreasing,
// and entries past the last used one repeat it.  With nothing masked this is
// jenks_group with 16 classes.
void jenks_group_masked(const float* vals, const uint8_t* keep, int n, uint8_t* codes,
                        uint16_t* book, JenksScratch& S) {
  float sub[128];
  int pos[128];
  int m = 0;
  for (int t = 0; t < n; ++t)
    if (keep[t]) {
      sub[m] = vals[t];
      pos[m] = t;
      ++m;
    }
  if (m == n) {
    jenks_group(vals, n, 16, codes, book, S);
    return;
  }
  const int k = std::min(15, m);
  uint8_t c[128];
  uint16_t cb[16];
  if (k > 0) jenks_group(sub, m, k, c, cb, S);
  int z = 0;
  while (z < k && (cb[z] & 0x8000u) && (cb[z] & 0x7fffu)) ++z;  // strictly negative
  for (int j = 0; j < z; ++j) book[j] = cb[j];
  book[z] = 0;
  for (int j = z; j < k; ++j) book[j + 1] = cb[j];
  for (int j = k + 1; j < 16; ++j) book[j] = book[k];
  for (int t = 0; t < n; ++t) codes[t] = (uint8_t)z;
  for (int i = 0; i < m; ++i) codes[pos[i]] = (uint8_t)(c[i] + (c[i] >= z ? 1 : 0));
}

// ---------------------------------------------------------------------------------
// E2M1 rounding: |q| onto {0,.5,1,1.5,2,3,4,6}, nearest, ties to even index, sat 6.
// ---------------------------------------------------------------------------------
uint8_t e2m1_index(double a) {
  static const double mids[7] = {0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0};
  int idx = 0;
  bool tie = false;
  for (int t = 0; t < 7; ++t) {
    if (a > mids[t]) ++idx;
    if (a == mids[t]) tie = true;
  }
  if (tie && (idx & 1)) ++idx;
  return (uint8_t)std::min(idx, 7);
}

bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

// Threads for the layout transforms (pure permutations): one per 64K items, at most the
// machine's hardware threads (and 16).
int layout_threads(int64_t items) {
  const int hw = (int)std::max(1u, std::thread::hardware_concurrency());
  return (int)std::max<int64_t>(1, std::min<int64_t>({items / 65536 + 1, hw, 16}));
}

}  // namespace

// ===================================================================================
// C ABI
// ===================================================================================
extern "C" {

int fb_abi_version(void) { return FB_ABI_VERSION; }

const char* fb_strerror(int code) {
  switch (code) {
    case FB_OK: return "ok";
    case FB_ERR_NULL: return "fourbit: required pointer is NULL";
    case FB_ERR_SHAPE: return "fourbit: N, K or B out of range (need N>=1, K>=128, K%128==0, B>=1)";
    case FB_ERR_GROUP: return "fourbit: group size must be 128 for GF4 and 32 for E2M1";
    case FB_ERR_FORMAT: return "fourbit: unknown format";
    case FB_ERR_DTYPE: return "fourbit: unsupported dtype (GF4 needs fp16 x; E2M1 fp16/bf16 x; y fp16/bf16/fp32)";
    case FB_ERR_FWHT:
      return "fourbit: fwht_block must be 0 or a power of two in [2, 4096] dividing K";
    case FB_ERR_ALIGN: return "fourbit: device pointers must be 16-byte aligned";
    case FB_ERR_WORKSPACE: return "fourbit: workspace smaller than fb_workspace_bytes()";
    case FB_ERR_BATCH: return "fourbit: batch size not supported by this entry point";
    case FB_ERR_VALUE: return "fourbit: non-finite weight or scale, non-positive scale, non-integer level, or a codebook entry beyond fp16 range";
    case FB_ERR_HIP: return "fourbit: HIP runtime call failed";
    case FB_ERR_THREADS: return "fourbit: nthreads must be >= 1";
    case FB_ERR_LDS: return "fourbit: activation vector does not fit the kernel's LDS budget";
    case FB_ERR_LEVELS: return "fourbit: the integer levels of a 128-group span more than 16 values";
    case FB_ERR_SCRATCH:
      return "fourbit: the shape needs more scratch than fb_gemv_noalloc's fixed 1 MiB device "
             "array (a rotated call of B*K > 524288 values); use fb_gemv with a workspace";
    default: return "fourbit: unknown error";
  }
}

int fb_validate(const fb_shape_t* s) {
  if (!s) return FB_ERR_NULL;
  if (s->fmt != FB_FMT_GF4 && s->fmt != FB_FMT_E2M1) return FB_ERR_FORMAT;
  if (s->N < 1 || s->K < 128 || s->K % 128 != 0 || s->B < 1) return FB_ERR_SHAPE;
  if (s->N > (1 << 26) || s->K > (1 << 24)) return FB_ERR_SHAPE;
  if ((int64_t)s->N * (s->K / 128) > INT32_MAX) return FB_ERR_SHAPE;  // < 2^31 groups
  if (s->fmt == FB_FMT_GF4 && s->group != 128) return FB_ERR_GROUP;
  if (s->fmt == FB_FMT_E2M1 && s->group != 32) return FB_ERR_GROUP;
  // the kernel's rotation has stages up to 4096 (12 butterfly levels)
  if (s->fwht_block != 0 && (!is_pow2(s->fwht_block) || s->fwht_block < 2 ||
                             s->fwht_block > 4096 || s->K % s->fwht_block != 0))
    return FB_ERR_FWHT;
  if (s->fmt == FB_FMT_GF4 && s->x_dtype != FB_DT_F16) return FB_ERR_DTYPE;
  if (s->fmt == FB_FMT_E2M1 && s->x_dtype != FB_DT_F16 && s->x_dtype != FB_DT_BF16)
    return FB_ERR_DTYPE;
  if (s->y_dtype != FB_DT_F16 && s->y_dtype != FB_DT_BF16 && s->y_dtype != FB_DT_F32)
    return FB_ERR_DTYPE;
  return FB_OK;
}

size_t fb_device_bytes(const fb_shape_t* s) {
  if (fb_validate(s) != FB_OK) return 0;
  return (size_t)fb::device_bytes(s->N, s->K, s->fmt);
}

int fb_quantize_gf4(const float* w, int32_t N, int32_t K, uint8_t* codes, uint16_t* codebook,
                    int32_t nthreads) {
  if (!w || !codes || !codebook) return FB_ERR_NULL;
  if (N < 1 || K < 128 || K % 128) return FB_ERR_SHAPE;
  if (nthreads < 1) return FB_ERR_THREADS;
  const int64_t total = (int64_t)N * K;
  for (int64_t t = 0; t < total; ++t)
    if (!std::isfinite(w[t])) return FB_ERR_VALUE;
  const int G = K / 128;
  parallel_for((int64_t)N * G, nthreads, [&](int64_t b, int64_t e) {
    JenksScratch S(128, 16);
    uint8_t c[128];
    for (int64_t it = b; it < e; ++it) {
      const int64_t n = it / G, g = it % G;
      jenks_group(w + n * K + g * 128, 128, 16, c, codebook + it * 16, S);
      uint8_t* dst = codes + n * (K / 2) + g * 64;
      for (int j = 0; j < 64; ++j) dst[j] = (uint8_t)(c[2 * j] | (c[2 * j + 1] << 4));
    }
  });
  return FB_OK;
}

int fb_quantize_gf4_masked(const float* w, const uint8_t* keep, int32_t N, int32_t K,
                           uint8_t* codes, uint16_t* codebook, int32_t nthreads) {
  if (!keep) return fb_quantize_gf4(w, N, K, codes, codebook, nthreads);
  if (!w || !codes || !codebook) return FB_ERR_NULL;
  if (N < 1 || K < 128 || K % 128) return FB_ERR_SHAPE;
  if (nthreads < 1) return FB_ERR_THREADS;
  const int64_t total = (int64_t)N * K;
  for (int64_t t = 0; t < total; ++t)
    if (keep[t] && !std::isfinite(w[t])) return FB_ERR_VALUE;
  const int G = K / 128;
  parallel_for((int64_t)N * G, nthreads, [&](int64_t b, int64_t e) {
    JenksScratch S(128, 16);
    uint8_t c[128];
    for (int64_t it = b; it < e; ++it) {
      const int64_t n = it / G, g = it % G;
      const int64_t off = n * K + g * 128;
      jenks_group_masked(w + off, keep + off, 128, c, codebook + it * 16, S);
      uint8_t* dst = codes + n * (K / 2) + g * 64;
      for (int j = 0; j < 64; ++j) dst[j] = (uint8_t)(c[2 * j] | (c[2 * j + 1] << 4));
    }
  });
  return FB_OK;
}

int fb_pack_levels_gf4(const float* levels, const float* scale, int32_t N, int32_t K,
                       uint8_t* codes, uint16_t* codebook, int32_t nthreads) {
  if (!levels || !scale || !codes || !codebook) return FB_ERR_NULL;
  if (N < 1 || K < 128 || K % 128) return FB_ERR_SHAPE;
  if (nthreads < 1) return FB_ERR_THREADS;
  for (int32_t n = 0; n < N; ++n)
    if (!(std::isfinite(scale[n]) && scale[n] > 0.0f)) return FB_ERR_VALUE;
  const int G = K / 128;
  std::atomic<int> status{FB_OK};
  parallel_for((int64_t)N * G, nthreads, [&](int64_t b, int64_t e) {
    for (int64_t it = b; it < e; ++it) {
      const int64_t n = it / G, g = it % G;
      const float* v = levels + n * K + g * 128;
      float lo = std::numeric_limits<float>::infinity(), hi = -lo;
      for (int t = 0; t < 128; ++t) {
        if (!std::isfinite(v[t]) || std::floor(v[t]) != v[t]) {
          status.store(FB_ERR_VALUE);
          return;
        }
        lo = std::min(lo, v[t]);
        hi = std::max(hi, v[t]);
      }
      lo += 0.0f;  // -0 -> +0, so a group of zeros has a +0 entry
      if (hi - lo > 15.0f) {
        status.store(FB_ERR_LEVELS);
        return;
      }
      const int used = (int)(hi - lo);
      uint16_t* bk = codebook + it * 16;
      for (int j = 0; j < 16; ++j) {
        const float lev = lo + (float)std::min(j, used);
        bk[j] = f32_to_f16_rne(scale[n] * lev);
        if ((bk[j] & 0x7fffu) >= 0x7c00u) {
          status.store(FB_ERR_VALUE);
          return;
        }
      }
      uint8_t* dst = codes + n * (K / 2) + g * 64;
      for (int j = 0; j < 64; ++j)
        dst[j] = (uint8_t)((int)(v[2 * j] - lo) | ((int)(v[2 * j + 1] - lo) << 4));
    }
  });
  return status.load();
}

int fb_quantize_e2m1(const float* w, int32_t N, int32_t K, uint8_t* codes, uint8_t* scales,
                     int32_t nthreads) {
  if (!w || !codes || !scales) return FB_ERR_NULL;
  if (N < 1 || K < 128 || K % 128) return FB_ERR_SHAPE;
  if (nthreads < 1) return FB_ERR_THREADS;
  const int64_t total = (int64_t)N * K;
  for (int64_t t = 0; t < total; ++t)
    if (!std::isfinite(w[t])) return FB_ERR_VALUE;
  const int G = K / 32;
  parallel_for((int64_t)N * G, nthreads, [&](int64_t b, int64_t e) {
    for (int64_t it = b; it < e; ++it) {
      const float* v = w + it * 32;  // rows are contiguous groups of 32
      float amax = 0.0f;
      for (int t = 0; t < 32; ++t) amax = std::max(amax, std::fabs(v[t]));
      int ex = 0;
      if (amax > 0.0f) {
        int e2;
        std::frexp((double)amax, &e2);  // amax = m * 2^e2, m in [0.5, 1)
        ex = std::min(127, std::max(-127, e2 - 1 - 2));
      }
      scales[it] = (uint8_t)(ex + 127);
      uint8_t c[32];
      for (int t = 0; t < 32; ++t) {
        const double q = std::ldexp((double)v[t], -ex);
        const uint8_t idx = e2m1_index(std::fabs(q));
        c[t] = (uint8_t)((std::signbit(v[t]) ? 8 : 0) | idx);
      }
      uint8_t* dst = codes + it * 16;
      for (int j = 0; j < 16; ++j) dst[j] = (uint8_t)(c[2 * j] | (c[2 * j + 1] << 4));
    }
  });
  return FB_OK;
}

int fb_fwht_rows_f32(float* w, int32_t N, int32_t K, int32_t block, int32_t nthreads) {
  if (!w) return FB_ERR_NULL;
  if (N < 1 || K < 1) return FB_ERR_SHAPE;
  if (!is_pow2(block) || block < 2 || K % block) return FB_ERR_FWHT;
  if (nthreads < 1) return FB_ERR_THREADS;
  const double sc = 1.0 / std::sqrt((double)block);
  parallel_for((int64_t)N, nthreads, [&](int64_t b, int64_t e) {
    std::vector<double> t(block);
    for (int64_t n = b; n < e; ++n) {
      for (int k0 = 0; k0 < K; k0 += block) {
        float* row = w + n * K + k0;
        for (int u = 0; u < block; ++u) t[u] = (double)row[u];
        for (int h = 1; h < block; h *= 2)
          for (int p = 0; p < block; p += 2 * h)
            for (int u = 0; u < h; ++u) {
              const double x = t[p + u], y = t[p + h + u];
              t[p + u] = x + y;
              t[p + h + u] = x - y;
            }
        for (int u = 0; u < block; ++u) row[u] = (float)(t[u] * sc);
      }
    }
  });
  return FB_OK;
}

int fb_to_device(const uint8_t* codes, const void* meta, void* wdev, const fb_shape_t* s) {
  if (!codes || !meta || !wdev) return FB_ERR_NULL;
  const int st = fb_validate(s);
  if (st != FB_OK) return st;
  const int64_t ipr = s->K / fb::kItemCodes;
  const int64_t items = (int64_t)s->N * ipr;
  std::memset(wdev, 0, fb_device_bytes(s));
  uint8_t* out = (uint8_t*)wdev;
  // items write disjoint bytes of the stream
  parallel_for(items, layout_threads(items), [&](int64_t b, int64_t e) {
    for (int64_t i = b; i < e; ++i) {
      const int64_t n = i / ipr, g = i % ipr;
      const uint8_t* crow = codes + n * (s->K / 2) + g * 64;  // 128 codes = 64 bytes
      if (s->fmt == FB_FMT_GF4) {
        const uint16_t* book = (const uint16_t*)meta + (n * ipr + g) * 16;
        fb::gf4_encode_item(crow, book, out, n, g, s->K);
      } else {
        const uint8_t* sc = (const uint8_t*)meta + (n * ipr + g) * 4;
        fb::e2m1_encode_item(crow, sc, out, n, g, s->K);
      }
    }
  });
  return FB_OK;
}

int fb_from_device(const void* wdev, uint8_t* codes, void* meta, const fb_shape_t* s) {
  if (!codes || !meta || !wdev) return FB_ERR_NULL;
  const int st = fb_validate(s);
  if (st != FB_OK) return st;
  const int64_t ipr = s->K / fb::kItemCodes;
  const int64_t items = (int64_t)s->N * ipr;
  const uint8_t* in = (const uint8_t*)wdev;
  parallel_for(items, layout_threads(items), [&](int64_t b, int64_t e) {
    for (int64_t i = b; i < e; ++i) {
      const int64_t n = i / ipr, g = i % ipr;
      uint8_t* crow = codes + n * (s->K / 2) + g * 64;
      if (s->fmt == FB_FMT_GF4) {
        uint16_t* book = (uint16_t*)meta + (n * ipr + g) * 16;
        fb::gf4_decode_item(in, n, g, s->K, crow, book);
      } else {
        uint8_t* sc = (uint8_t*)meta + (n * ipr + g) * 4;
        fb::e2m1_decode_item(in, n, g, s->K, crow, sc);
      }
    }
  });
  return FB_OK;
}

int fb_dequant_host(const uint8_t* codes, const void* meta, float* w_out, const fb_shape_t* s) {
  if (!codes || !meta || !w_out) return FB_ERR_NULL;
  const int st = fb_validate(s);
  if (st != FB_OK) return st;
  const int64_t N = s->N, K = s->K;
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k) {
      const int c = (codes[n * (K / 2) + k / 2] >> ((k & 1) * 4)) & 15;
      float v;
      if (s->fmt == FB_FMT_GF4) {
        const uint16_t h = ((const uint16_t*)meta)[(n * (K / 128) + k / 128) * 16 + c];
        v = f16_bits_to_f32(h);
      } else {
        static const float grid[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
        const int e = (int)((const uint8_t*)meta)[n * (K / 32) + k / 32] - 127;
        v = std::ldexp((c & 8) ? -grid[c & 7] : grid[c & 7], e);
      }
      w_out[n * K + k] = v;
    }
  return FB_OK;
}

}  // extern "C"

namespace {

// The within-class SSD of every split of n values taken in the order given (1 <= n < 2^31):
// visit(i, ssd(i)) for i = 0, 1, ..., n - 1 in turn.  fp64 sums in a fixed association order
// -- centre c = srt[n / 2]; d = srt - c and d * d; prefix sums sequential within blocks of
// 256, block totals sequential within superblocks of 256 blocks, superblock totals sequential
// -- the same arithmetic, in the same order, as fourbit_jenks2.hip, so that host and GPU
// give the same bits.  T: float or double values.
template <typename T, typename Visit>
void jenks2_ssd_sorted(const T* srt, int64_t n, Visit&& visit) {
  constexpr int64_t kBlk = 256, kSup = 256;
  const double c = (double)srt[n / 2];
  const int64_t nblk = (n + kBlk - 1) / kBlk, nsup = (nblk + kSup - 1) / kSup;
  std::vector<double> t1(nblk), t2(nblk), bx1(nblk), bx2(nblk), sx1(nsup + 1), sx2(nsup + 1);
  for (int64_t b = 0; b < nblk; ++b) {
    double a1 = 0.0, a2 = 0.0;
    for (int64_t i = b * kBlk; i < std::min(n, b * kBlk + kBlk); ++i) {
      const double d = (double)srt[i] - c;
      const double q = d * d;
      a1 = a1 + d;
      a2 = a2 + q;
    }
    t1[b] = a1;
    t2[b] = a2;
  }
  std::vector<double> u1(nsup), u2(nsup);
  for (int64_t s = 0; s < nsup; ++s) {
    double a1 = 0.0, a2 = 0.0;
    for (int64_t b = s * kSup; b < std::min(nblk, s * kSup + kSup); ++b) {
      bx1[b] = a1;
      bx2[b] = a2;
      a1 = a1 + t1[b];
      a2 = a2 + t2[b];
    }
    u1[s] = a1;
    u2[s] = a2;
  }
  {
    double a1 = 0.0, a2 = 0.0;
    for (int64_t s = 0; s < nsup; ++s) {
      sx1[s] = a1;
      sx2[s] = a2;
      a1 = a1 + u1[s];
      a2 = a2 + u2[s];
    }
    sx1[nsup] = a1;
    sx2[nsup] = a2;
  }
  const double pt = sx1[nsup], qt = sx2[nsup];
  for (int64_t b = 0; b < nblk; ++b) {
    const double base1 = sx1[b / kSup] + bx1[b], base2 = sx2[b / kSup] + bx2[b];
    double l1 = 0.0, l2 = 0.0;
    for (int64_t i = b * kBlk; i < std::min(n, b * kBlk + kBlk); ++i) {
      const double p = base1 + l1, q = base2 + l2;
      const double left = i == 0 ? 0.0 : q - (p * p) / (double)i;
      const double rp = pt - p;
      const double right = (qt - q) - (rp * rp) / (double)(n - i);
      visit(i, left + right);
      const double d = (double)srt[i] - c;
      const double dq = d * d;
      l1 = l1 + d;
      l2 = l2 + dq;
    }
  }
}

// Two-class natural breaks over one array of n finite values (1 <= n < 2^31): the stable
// ascending order, the SSD of every split of it (jenks2_ssd_sorted), the first minimum.  The
// same bits as fb_jenks2_gpu and the filter kernels of fourbit_jenks2.hip.
void jenks2_one(const float* w, int64_t n, uint8_t* keep, int64_t* split, double* gvf) {
  std::vector<int> order((size_t)n);
  std::iota(order.begin(), order.end(), 0);
  // ascending, stable by index; -0.0 == +0.0 under <
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return w[a] < w[b]; });
  std::vector<float> srt((size_t)n);
  for (int64_t t = 0; t < n; ++t) srt[t] = w[order[t]];
  double best = 0.0, ssd0 = 0.0;
  int64_t arg = -1;
  jenks2_ssd_sorted(srt.data(), n, [&](int64_t i, double v) {
    if (arg < 0 || v < best) {
      best = v;
      arg = i;
    }
    if (i == 0) ssd0 = v;
  });
  for (int64_t t = 0; t < n; ++t) keep[order[t]] = t >= arg ? 1 : 0;
  *split = arg;
  *gvf = (ssd0 - best) / (ssd0 + 1e-8);
}

// ssd[i] (in T) of every split of srt[0 .. n) in the order given.
template <typename T>
void jenks2_ssd_out(const T* srt, int64_t n, T* ssd) {
  jenks2_ssd_sorted(srt, n, [&](int64_t i, double v) { ssd[i] = (T)v; });
}

}  // namespace

extern "C" {

// The whole array (the reference's Linear_Mask / Bias_Mask, cuda_helpers.py:378-411).
int fb_jenks2_host(const float* w, int64_t n, uint8_t* keep, int64_t* split, double* gvf) {
  if (!w || !keep || !split || !gvf) return FB_ERR_NULL;
  if (n < 1 || n > INT32_MAX) return FB_ERR_SHAPE;
  for (int64_t t = 0; t < n; ++t)
    if (!std::isfinite(w[t])) return FB_ERR_VALUE;
  jenks2_one(w, n, keep, split, gvf);
  return FB_OK;
}

// The per-split SSD of a pre-sorted array (the reference's jenks_optimization_cuda and
// jenks_optimization_biases_cuda, cuda_helpers.py:187-211, :122-146), in its dtype.
int fb_jenks2_ssd_host(const void* sorted, int64_t n, int32_t dtype, void* ssd) {
  if (!sorted || !ssd) return FB_ERR_NULL;
  if (n < 1 || n > INT32_MAX) return FB_ERR_SHAPE;
  if (dtype == FB_DT_F32)
    jenks2_ssd_out(static_cast<const float*>(sorted), n, static_cast<float*>(ssd));
  else if (dtype == FB_DT_F64)
    jenks2_ssd_out(static_cast<const double*>(sorted), n, static_cast<double*>(ssd));
  else
    return FB_ERR_DTYPE;
  return FB_OK;
}

// The same for every filter on its own (jenks_optimization_cuda_conv, :258-289).
int fb_jenks2_ssd_filters_host(const void* sorted, int64_t nf, int32_t n, int32_t dtype,
                               void* ssd, int32_t nthreads) {
  if (!sorted || !ssd) return FB_ERR_NULL;
  if (nf < 1 || n < 1 || n > FB_JENKS2_FILTER_MAX || nf > INT32_MAX) return FB_ERR_SHAPE;
  if (dtype != FB_DT_F32 && dtype != FB_DT_F64) return FB_ERR_DTYPE;
  if (nthreads < 1) return FB_ERR_THREADS;
  parallel_for(nf, nthreads, [&](int64_t b, int64_t e) {
    for (int64_t f = b; f < e; ++f) {
      if (dtype == FB_DT_F32)
        jenks2_ssd_out(static_cast<const float*>(sorted) + f * n, n,
                       static_cast<float*>(ssd) + f * n);
      else
        jenks2_ssd_out(static_cast<const double*>(sorted) + f * n, n,
                       static_cast<double*>(ssd) + f * n);
    }
  });
  return FB_OK;
}

// Every filter on its own (the reference's Conv_Mask, cuda_helpers.py:333-376): filter f is
// w[f n .. f n + n), as a [out, in, kh, kw] weight's (out, in) slices are.
int fb_jenks2_filters_host(const float* w, int64_t nf, int32_t n, uint8_t* keep, int32_t* split,
                           double* gvf, int32_t nthreads) {
  if (!w || !keep || !split || !gvf) return FB_ERR_NULL;
  if (nf < 1 || n < 1 || n > FB_JENKS2_FILTER_MAX || nf > INT32_MAX) return FB_ERR_SHAPE;
  if (nthreads < 1) return FB_ERR_THREADS;
  const int64_t total = nf * n;
  for (int64_t t = 0; t < total; ++t)
    if (!std::isfinite(w[t])) return FB_ERR_VALUE;
  parallel_for(nf, nthreads, [&](int64_t b, int64_t e) {
    for (int64_t f = b; f < e; ++f) {
      int64_t sp = 0;
      jenks2_one(w + f * n, n, keep + f * n, &sp, gvf + f);
      split[f] = (int32_t)sp;
    }
  });
  return FB_OK;
}

}  // extern "C"
