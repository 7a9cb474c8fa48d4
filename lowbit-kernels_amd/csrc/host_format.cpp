// Host-side (CPU memory) format functions: the C++ counterparts of the reference's lowbit/quant.py, used by the
// Python `lowbit.quant` module. They are not on the GPU path; they let a caller pack weights without a GPU, exactly as
// the reference's numpy golden model does, bit for bit.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "lowbit_w4.h"
#include "status.hpp"

namespace {

// IEEE binary32 -> binary16, round to nearest even (numpy's astype(float16) rule)
uint16_t f32_to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);          // >= 65520 rounds to infinity
  if (ax < 0x38800000u) {                                             // below 2^-14: subnormal or zero
    float v;
    std::memcpy(&v, &ax, 4);
    return (uint16_t)(sign | (uint32_t)std::nearbyint(v * 16777216.0f));   // exact scaling, then round half even
  }
  const uint32_t mant = ax & 0x7FFFFFu;
  uint32_t h = ((((ax >> 23) - 127u + 15u)) << 10) | (mant >> 13);
  const uint32_t rem = mant & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;             // a carry moves into the exponent correctly
  return (uint16_t)(sign | h);
}

float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  float v;
  if (e == 0) {
    v = std::ldexp((float)m, -24);
  } else if (e == 31) {
    uint32_t bits = 0x7F800000u | (m << 13);
    std::memcpy(&v, &bits, 4);
  } else {
    uint32_t bits = ((e - 15u + 127u) << 23) | (m << 13);
    std::memcpy(&v, &bits, 4);
  }
  uint32_t b;
  std::memcpy(&b, &v, 4);
  b |= sign;
  std::memcpy(&v, &b, 4);
  return v;
}

uint32_t canonical_to_v3(uint32_t w) {
  uint32_t e = w & 0x0F0F0F0Fu, o = (w >> 4) & 0x0F0F0F0Fu;
  e = (e | (e >> 4)) & 0x00FF00FFu;
  e = (e | (e >> 8)) & 0x0000FFFFu;
  o = (o | (o >> 4)) & 0x00FF00FFu;
  o = (o | (o >> 8)) & 0x0000FFFFu;
  return e | (o << 16);
}

template <typename F>
void parallel_rows(int64_t N, int64_t work_per_row, F&& fn) {
  const int64_t total = N * work_per_row;
  unsigned threads = std::thread::hardware_concurrency();
  if (threads == 0) threads = 1;
  if (threads > 32) threads = 32;
  if (total < (1 << 20) || threads == 1 || N < 2) {
    fn(0, N);
    return;
  }
  if ((int64_t)threads > N) threads = (unsigned)N;
  std::vector<std::thread> pool;
  const int64_t per = (N + threads - 1) / threads;
  for (unsigned t = 0; t < threads; ++t) {
    const int64_t a = t * per, b = std::min<int64_t>(N, a + per);
    if (a < b) pool.emplace_back([&, a, b] { fn(a, b); });
  }
  for (auto& th : pool) th.join();
}

int check_group(int64_t K, int64_t group) {
  if (group <= 0 || group % 32 || K % group)
    return lowbit::fail(LOWBIT_ERR_GROUP, "K=%lld must be a multiple of the group size %lld, itself a multiple of 32",
                        (long long)K, (long long)group);
  return LOWBIT_OK;
}

}  // namespace

extern "C" int lowbit_host_quantize(const float* w, uint8_t* packed, uint16_t* scales, int64_t N, int64_t K,
                                    int64_t group) {
  if (!w || !packed || !scales) return lowbit::fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (N < 0 || K <= 0) return lowbit::fail(LOWBIT_ERR_SHAPE, "shape mismatch");
  if (int rc = check_group(K, group)) return rc;
  const int64_t KG = K / group;
  parallel_rows(N, K, [&](int64_t r0, int64_t r1) {
    for (int64_t n = r0; n < r1; ++n) {
      for (int64_t g = 0; g < KG; ++g) {
        const float* v = w + n * K + g * group;
        float amax = 0.f;
        for (int64_t i = 0; i < group; ++i) amax = std::max(amax, std::fabs(v[i]));
        uint16_t sh = f32_to_f16(amax / 7.0f);
        if ((sh & 0x7FFFu) == 0) sh = 0x3C00u;                       // an all-zero group: scale 1.0
        scales[n * KG + g] = sh;
        const float sf = f16_to_f32(sh);
        for (int64_t i = 0; i < group; i += 2) {
          const float q0 = std::fmin(std::fmax(std::nearbyint(v[i] / sf), -8.f), 7.f);
          const float q1 = std::fmin(std::fmax(std::nearbyint(v[i + 1] / sf), -8.f), 7.f);
          packed[(n * K + g * group + i) / 2] = (uint8_t)((uint32_t)(q0 + 8.f) | ((uint32_t)(q1 + 8.f) << 4));
        }
      }
    }
  });
  return LOWBIT_OK;
}

extern "C" int lowbit_host_unpack(const uint8_t* packed, int8_t* out, int64_t N, int64_t K) {
  if (!packed || !out) return lowbit::fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (N < 0 || K < 0 || K % 2) return lowbit::fail(LOWBIT_ERR_SHAPE, "shape mismatch");
  for (int64_t i = 0; i < N * K / 2; ++i) {
    out[2 * i] = (int8_t)((packed[i] & 0x0F) - 8);
    out[2 * i + 1] = (int8_t)((packed[i] >> 4) - 8);
  }
  return LOWBIT_OK;
}

extern "C" int lowbit_host_dequantize(const uint8_t* packed, const uint16_t* scales, float* out, int64_t N, int64_t K,
                                      int64_t group) {
  if (!packed || !scales || !out) return lowbit::fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (N < 0 || K <= 0) return lowbit::fail(LOWBIT_ERR_SHAPE, "shape mismatch");
  if (K % group || group <= 0) return lowbit::fail(LOWBIT_ERR_GROUP, "K=%lld must be a multiple of the group size %lld",
                                                   (long long)K, (long long)group);
  const int64_t KG = K / group;
  parallel_rows(N, K, [&](int64_t r0, int64_t r1) {
    for (int64_t n = r0; n < r1; ++n)
      for (int64_t k = 0; k < K; ++k) {
        const uint8_t b = packed[(n * K + k) / 2];
        const int q = ((k & 1) ? (b >> 4) : (b & 0x0F)) - 8;
        out[n * K + k] = (float)q * f16_to_f32(scales[n * KG + k / group]);
      }
  });
  return LOWBIT_OK;
}

extern "C" int lowbit_host_relayout(const uint8_t* src, uint8_t* dst, int64_t N, int64_t K, int layout) {
  if (!src || !dst) return lowbit::fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (src == dst) return lowbit::fail(LOWBIT_ERR_ARG, "dst must not alias src");
  if (N < 0 || K < 0 || K % 8) return lowbit::fail(LOWBIT_ERR_SHAPE, "K=%lld must be a multiple of 8", (long long)K);
  const int64_t half_k = K / 2, words = K / 8;
  if (layout == LOWBIT_LAYOUT_V3) {
    for (int64_t i = 0; i < N * words; ++i) {
      uint32_t w;
      std::memcpy(&w, src + 4 * i, 4);
      w = canonical_to_v3(w);
      std::memcpy(dst + 4 * i, &w, 4);
    }
    return LOWBIT_OK;
  }
  if (layout == LOWBIT_LAYOUT_NV_MMA || layout == LOWBIT_LAYOUT_MFMA) {
    if (K % 128)
      return lowbit::fail(LOWBIT_ERR_LAYOUT, "K=%lld must be a multiple of 128 for the %s layout", (long long)K,
                          layout == LOWBIT_LAYOUT_MFMA ? "MFMA" : "tensor-core");
    const int64_t chunks = half_k / 64;
    for (int64_t n = 0; n < N; ++n)
      for (int64_t c = 0; c < chunks; ++c) {
        uint8_t tmp[64];
        const uint8_t* in = src + n * half_k + 64 * c;
        if (layout == LOWBIT_LAYOUT_NV_MMA) {
          // byte 16 t + s of a chunk holds canonical byte 4 s + t (reference lowbit/quant.py:67-68)
          for (int t = 0; t < 4; ++t)
            for (int s = 0; s < 16; ++s) tmp[16 * t + s] = in[4 * s + t];
        } else {
          std::memcpy(tmp, in, 64);
        }
        for (int j = 0; j < 16; ++j) {
          uint32_t w;
          std::memcpy(&w, tmp + 4 * j, 4);
          w = canonical_to_v3(w);
          std::memcpy(tmp + 4 * j, &w, 4);
        }
        int64_t off;
        if (layout == LOWBIT_LAYOUT_NV_MMA) {
          off = n * half_k + 64 * c;
        } else {
          const int64_t t = n / 16, r = n % 16, rows = std::min<int64_t>(16, N - 16 * t);
          off = t * 16 * half_k + c * rows * 64 + 64 * r;
        }
        std::memcpy(dst + off, tmp, 64);
      }
    return LOWBIT_OK;
  }
  return lowbit::fail(LOWBIT_ERR_ARG, "unknown layout %d", layout);
}

extern "C" int lowbit_host_gemv_reference(const double* x, const uint8_t* packed, const uint16_t* scales, double* y,
                                          int64_t M, int64_t N, int64_t K, int64_t group) {
  if (!x || !packed || !scales || !y) return lowbit::fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (M < 0 || N < 0 || K <= 0) return lowbit::fail(LOWBIT_ERR_SHAPE, "shape mismatch");
  if (K % group || group <= 0) return lowbit::fail(LOWBIT_ERR_GROUP, "K=%lld must be a multiple of the group size %lld",
                                                   (long long)K, (long long)group);
  const int64_t KG = K / group;
  parallel_rows(N, K * (M > 0 ? M : 1), [&](int64_t r0, int64_t r1) {
    std::vector<double> wrow(K);
    for (int64_t n = r0; n < r1; ++n) {
      for (int64_t k = 0; k < K; ++k) {
        const uint8_t b = packed[(n * K + k) / 2];
        const int q = ((k & 1) ? (b >> 4) : (b & 0x0F)) - 8;
        wrow[k] = (double)q * (double)f16_to_f32(scales[n * KG + k / group]);
      }
      for (int64_t m = 0; m < M; ++m) {
        double acc = 0.0;
        for (int64_t k = 0; k < K; ++k) acc += x[m * K + k] * wrow[k];
        y[m * N + n] = acc;
      }
    }
  });
  return LOWBIT_OK;
}
