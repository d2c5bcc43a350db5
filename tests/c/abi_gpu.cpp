// A native caller of libfourbit's GPU entry point, with no Python or torch: device buffers
// from hipMalloc, a stream from hipStreamCreate, weights packed by the host packers and
// laid out by fb_to_device, fb_gemv launched on that stream, and y checked against an
// fp64 host product of the exact host decode (fb_dequant_host) with the activations
// rounded as the kernel reads them.  Bound: |err| <= 1e-2 + 1e-3 |ref|, plus half an
// output ulp for an fp16 y.
// Cases: GF4, fp16 x, fp32 y, batch 3, N = 300 (the last row tile is partial);
//        E2M1, bf16 x, fp16 y, batch 16, K = 2048 (the MFMA columns are all live);
//        E2M1, bf16 x, fp32 y, batch 8, on the native FP4 path (fb_gemv_mx, with its
//        workspace from hipMalloc).
// Built by if_i_could_turn_back_time_amd/build_lib.py next to libfourbit.so; run by
// tests/test_gpu.py::test_c_abi_gpu_caller.  Prints one line per case and "ok".
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "fourbit.h"

#define HIP_OK(expr)                                                              \
  do {                                                                            \
    hipError_t e_ = (expr);                                                       \
    if (e_ != hipSuccess) {                                                       \
      std::fprintf(stderr, "%s: %s\n", #expr, hipGetErrorString(e_));             \
      std::exit(2);                                                               \
    }                                                                             \
  } while (0)

#define FB_OK_OR_DIE(expr)                                                        \
  do {                                                                            \
    int r_ = (expr);                                                              \
    if (r_ != FB_OK) {                                                            \
      std::fprintf(stderr, "%s: %s\n", #expr, fb_strerror(r_));                   \
      std::exit(2);                                                               \
    }                                                                             \
  } while (0)

static uint16_t to_f16(float f, float* back) {
  const _Float16 h = (_Float16)f;
  *back = (float)h;
  uint16_t b;
  std::memcpy(&b, &h, 2);
  return b;
}

static uint16_t to_bf16(float f, float* back) {  // round to nearest even (finite inputs)
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7FFFu + ((u >> 16) & 1u);
  const uint16_t b = (uint16_t)(u >> 16);
  const uint32_t v = (uint32_t)b << 16;
  std::memcpy(back, &v, 4);
  return b;
}

static float from_f16(uint16_t b) {
  _Float16 h;
  std::memcpy(&h, &b, 2);
  return (float)h;
}

// Returns the number of outputs outside the bound.
static int run_case(int fmt, int N, int K, int B, int x_dtype, int y_dtype, hipStream_t st,
                    bool mx = false) {
  std::mt19937 gen(1234 + fmt * 100 + B);
  std::normal_distribution<float> nd(0.0f, 1.0f);
  std::vector<float> w((size_t)N * K);
  for (auto& v : w) v = 0.02f * nd(gen);

  const int group = fmt == FB_FMT_GF4 ? 128 : 32;
  fb_shape_t s = {N, K, B, group, fmt, 0, x_dtype, y_dtype};
  FB_OK_OR_DIE(fb_validate(&s));
  std::vector<uint8_t> codes((size_t)N * K / 2);
  std::vector<uint8_t> meta(fmt == FB_FMT_GF4 ? (size_t)N * (K / 128) * 32 : (size_t)N * (K / 32));
  if (fmt == FB_FMT_GF4)
    FB_OK_OR_DIE(fb_quantize_gf4(w.data(), N, K, codes.data(),
                                 reinterpret_cast<uint16_t*>(meta.data()), 4));
  else
    FB_OK_OR_DIE(fb_quantize_e2m1(w.data(), N, K, codes.data(), meta.data(), 4));
  std::vector<float> wd((size_t)N * K);
  FB_OK_OR_DIE(fb_dequant_host(codes.data(), meta.data(), wd.data(), &s));
  std::vector<uint8_t> stream_bytes(fb_device_bytes(&s));
  FB_OK_OR_DIE(fb_to_device(codes.data(), meta.data(), stream_bytes.data(), &s));

  // activations, rounded as the kernel reads them
  std::vector<uint16_t> xb((size_t)B * K);
  std::vector<float> xr((size_t)B * K);
  for (size_t i = 0; i < xb.size(); ++i) {
    const float v = nd(gen);
    xb[i] = x_dtype == FB_DT_F16 ? to_f16(v, &xr[i]) : to_bf16(v, &xr[i]);
  }
  const size_t ysize = y_dtype == FB_DT_F32 ? 4 : 2;

  void *d_w = nullptr, *d_x = nullptr, *d_y = nullptr;
  HIP_OK(hipMalloc(&d_w, stream_bytes.size()));
  HIP_OK(hipMalloc(&d_x, xb.size() * 2));
  HIP_OK(hipMalloc(&d_y, (size_t)B * N * ysize));
  HIP_OK(hipMemcpyAsync(d_w, stream_bytes.data(), stream_bytes.size(), hipMemcpyHostToDevice, st));
  HIP_OK(hipMemcpyAsync(d_x, xb.data(), xb.size() * 2, hipMemcpyHostToDevice, st));
  void* d_ws = nullptr;
  const size_t ws_bytes = mx ? fb_mx_workspace_bytes(&s) : 0;
  if (mx) {
    if (!ws_bytes) {
      std::fprintf(stderr, "fb_mx_workspace_bytes: 0 for this shape\n");
      std::exit(2);
    }
    HIP_OK(hipMalloc(&d_ws, ws_bytes));  // hipMalloc gives 256-byte alignment
    FB_OK_OR_DIE(fb_gemv_mx(d_w, d_x, d_y, &s, d_ws, ws_bytes, st));
  } else {
    FB_OK_OR_DIE(fb_gemv(d_w, d_x, d_y, &s, nullptr, 0, st));
  }
  std::vector<uint8_t> yb((size_t)B * N * ysize);
  HIP_OK(hipMemcpyAsync(yb.data(), d_y, yb.size(), hipMemcpyDeviceToHost, st));
  HIP_OK(hipStreamSynchronize(st));
  HIP_OK(hipFree(d_w));
  HIP_OK(hipFree(d_x));
  HIP_OK(hipFree(d_y));
  if (d_ws) HIP_OK(hipFree(d_ws));

  int bad = 0;
  double emax = 0.0;
  for (int b = 0; b < B; ++b)
    for (int n = 0; n < N; ++n) {
      double ref = 0.0;
      for (int k = 0; k < K; ++k) ref += (double)wd[(size_t)n * K + k] * xr[(size_t)b * K + k];
      double y;
      double bound = 1e-2 + 1e-3 * std::fabs(ref);
      if (y_dtype == FB_DT_F32) {
        float f;
        std::memcpy(&f, &yb[((size_t)b * N + n) * 4], 4);
        y = f;
      } else {
        uint16_t h;
        std::memcpy(&h, &yb[((size_t)b * N + n) * 2], 2);
        y = from_f16(h);
        bound += std::ldexp(std::fabs(ref), -11);
      }
      const double err = std::fabs(y - ref);
      if (!(err <= bound)) ++bad;
      if (err > emax) emax = err;
    }
  std::printf("%s%s N=%d K=%d B=%d: max abs err %.3g, %d outside the bound\n",
              fmt == FB_FMT_GF4 ? "gf4" : "e2m1", mx ? " (fp4 mfma)" : "", N, K, B, emax, bad);
  return bad;
}

int main() {
  int dev_count = 0;
  HIP_OK(hipGetDeviceCount(&dev_count));
  if (dev_count < 1) {
    std::fprintf(stderr, "no GPU\n");
    return 2;
  }
  hipStream_t st;
  HIP_OK(hipStreamCreate(&st));
  int bad = run_case(FB_FMT_GF4, 300, 1024, 3, FB_DT_F16, FB_DT_F32, st);
  bad += run_case(FB_FMT_E2M1, 256, 2048, 16, FB_DT_BF16, FB_DT_F16, st);
  bad += run_case(FB_FMT_E2M1, 200, 4096, 8, FB_DT_BF16, FB_DT_F32, st, true);
  HIP_OK(hipStreamDestroy(st));
  if (bad) return 1;
  std::printf("ok\n");
  return 0;
}
