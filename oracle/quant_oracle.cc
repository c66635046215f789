// CPU oracle for weight rows: dequantization and the matvec twin. TEST INFRASTRUCTURE ONLY.
//
// A C++ restatement of crates/qwen36/src/quant.rs (WType::block / row_bytes at 60-74,
// dequant_row at 77-104, q8_0_block 161-167, scale_min_k4 170-179, q4k_block 182-206,
// q5k_block 209-228, q6k_block 231-252): ggml's block layouts for the six weight types the
// reference accepts, dequantized in the same f32 operations and order (products rounded before
// the subtraction; the build keeps every product unfused). Only tests/ load it, as the checker
// for the GPU's embed_rows, matvec and head_argmax.
//
// oc_matvec restates the twin of the matvec kernels (crates/kernels/src/twin/matvec.rs:21-131,
// twin/mod.rs:15-25), which the reference's GPU matvec equals bit for bit
// (crates/kernels/tests/gpu_kernels.rs:112-140).
//
// Pinned by (tests/test_oracle_quant.py): the reference's gguf-py rows of each type
// (crates/qwen36/tests/fixtures, checked at the reference's own 1e-6 tolerance and counted bit
// for bit), its hand-built blocks (quant.rs:266-409), numpy's own f16 conversion for every f16
// bit pattern, and row_bytes' table (quant.rs:270-277). oc_matvec: integer-valued rows and inputs
// whose every sum is exact (so any order gives the exact dot product, which numpy computes), the f64
// dot product of the dequantized row within the f32 sums' error bound, and lane partials whose
// tree order is visible in the result.
#include "sampler_oracle.h"

#include <cmath>
#include <cstring>

namespace {

// Elements and bytes per block, by the reference's type codes (quant.glsl:2-8): F32, BF16, Q8_0,
// Q4_K, Q5_K, Q6_K.
const uint32_t kPer[6] = {1, 1, 32, 256, 256, 256};
const uint32_t kBytes[6] = {4, 2, 34, 144, 176, 210};

// IEEE binary16 to f32, exactly (every f16 is an f32): sign, 5-bit exponent, 10-bit fraction.
float half_to_float(uint16_t h) {
  const uint32_t sign = (h >> 15) & 1u, exp = (h >> 10) & 31u, frac = h & 1023u;
  float v;
  if (exp == 0) {
    v = std::ldexp((float)frac, -24);  // subnormal (or zero)
  } else if (exp == 31) {
    v = frac ? NAN : INFINITY;
  } else {
    v = std::ldexp((float)(frac | 1024u), (int)exp - 25);
  }
  return sign ? -v : v;
}

float half_at(const uint8_t* b, size_t i) { return half_to_float((uint16_t)(b[i] | (b[i + 1] << 8))); }

// quant.rs:170-179 (ggml's get_scale_min_k4).
void scale_min_k4(uint32_t j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

// quant.rs:161-167.
void q8_0_block(const uint8_t* b, float* out) {
  const float d = half_at(b, 0);
  for (int i = 0; i < 32; ++i) out[i] = d * (float)(int8_t)b[2 + i];
}

// quant.rs:182-228: Q4_K (qh == nullptr) and Q5_K.
void k4_block(const uint8_t* b, const uint8_t* qh, const uint8_t* qs, float* out) {
  const float d = half_at(b, 0), dmin = half_at(b, 2);
  const uint8_t* scales = b + 4;
  for (uint32_t c = 0; c < 4; ++c) {
    uint8_t sc1, m1, sc2, m2;
    scale_min_k4(2 * c, scales, &sc1, &m1);
    scale_min_k4(2 * c + 1, scales, &sc2, &m2);
    const float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
    const float d2 = d * (float)sc2, mm2 = dmin * (float)m2;
    const uint8_t u1 = (uint8_t)(1u << (2 * c)), u2 = (uint8_t)(2u << (2 * c));
    for (uint32_t l = 0; l < 32; ++l) {
      const uint8_t q = qs[32 * c + l];
      const uint32_t h1 = (qh && (qh[l] & u1)) ? 16u : 0u, h2 = (qh && (qh[l] & u2)) ? 16u : 0u;
      const float p1 = d1 * (float)((q & 0xF) + h1);
      const float p2 = d2 * (float)((q >> 4) + h2);
      out[64 * c + l] = p1 - mm1;
      out[64 * c + 32 + l] = p2 - mm2;
    }
  }
}

// quant.rs:231-252.
void q6k_block(const uint8_t* b, float* out) {
  const float d = half_at(b, 208);
  for (uint32_t n = 0; n < 2; ++n) {
    const uint8_t *ql = b + 64 * n, *qh = b + 128 + 32 * n, *sc = b + 192 + 8 * n;
    float* y = out + 128 * n;
    for (uint32_t l = 0; l < 32; ++l) {
      const uint32_t is = l / 16;
      const int q1 = (int)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
      const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
      const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
      const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
      const float s1 = d * (float)(int8_t)sc[is], s2 = d * (float)(int8_t)sc[is + 2];
      const float s3 = d * (float)(int8_t)sc[is + 4], s4 = d * (float)(int8_t)sc[is + 6];
      y[l] = s1 * (float)q1;
      y[l + 32] = s2 * (float)q2;
      y[l + 64] = s3 * (float)q3;
      y[l + 96] = s4 * (float)q4;
    }
  }
}

// crates/kernels/src/twin/matvec.rs:21-84 (unit_dot): sum of w * x over 32-value unit u of a row,
// in the twin's f32 operations (each product rounded, then added, in order from 0).
float unit_dot(uint32_t t, const uint8_t* row, uint64_t u, const float* xs) {
  const float* x = xs + 32 * u;
  switch (t) {
    case 0: {
      const uint8_t* w = row + 128 * u;
      float s = 0.0f;
      for (int i = 0; i < 32; ++i) {
        float v;
        std::memcpy(&v, w + 4 * i, 4);
        const float p = v * x[i];
        s = s + p;
      }
      return s;
    }
    case 1: {
      const uint8_t* w = row + 64 * u;
      float s = 0.0f;
      for (int i = 0; i < 32; ++i) {
        const uint32_t bits = (uint32_t)(w[2 * i] | (w[2 * i + 1] << 8)) << 16;
        float v;
        std::memcpy(&v, &bits, 4);
        const float p = v * x[i];
        s = s + p;
      }
      return s;
    }
    case 2: {
      const uint8_t* b = row + 34 * u;
      float s = 0.0f;
      for (int i = 0; i < 32; ++i) {
        const float p = (float)(int8_t)b[2 + i] * x[i];
        s = s + p;
      }
      return half_at(b, 0) * s;
    }
    case 3:
    case 4: {
      const bool q5 = t == 4;
      const uint32_t bsz = q5 ? 176 : 144;
      const uint8_t* b = row + bsz * (u / 8);
      const uint32_t j = (uint32_t)(u % 8), c = j / 2, sh = 4 * (j % 2);
      uint8_t sc, mn;
      scale_min_k4(j, b + 4, &sc, &mn);
      const uint8_t* qs = b + (q5 ? 48 : 16) + 32 * c;
      float sq = 0.0f, sx = 0.0f;
      for (int l = 0; l < 32; ++l) {
        uint32_t q = (qs[l] >> sh) & 0xF;
        if (q5 && ((b[16 + l] >> j) & 1)) q += 16;
        const float p = (float)q * x[l];
        sq = sq + p;
        sx = sx + x[l];
      }
      const float a = (half_at(b, 0) * (float)sc) * sq;
      const float m = (half_at(b, 2) * (float)mn) * sx;
      return a - m;
    }
    default: {
      const uint8_t* b = row + 210 * (u / 8);
      const uint32_t j = (uint32_t)(u % 8), n = j / 4, m = j % 4;
      const uint8_t *ql = b + 64 * n + 32 * (m & 1), *qh = b + 128 + 32 * n;
      const uint32_t shl = 4 * (m >> 1), shh = 2 * m;
      float sa = 0.0f, sb = 0.0f;
      for (int l = 0; l < 32; ++l) {
        const uint32_t lo = (ql[l] >> shl) & 0xF, hi = (qh[l] >> shh) & 3;
        const float p = (float)((int)(lo | (hi << 4)) - 32) * x[l];
        if (l < 16) sa = sa + p;
        else sb = sb + p;
      }
      const float sca = (float)(int8_t)b[192 + 8 * n + 2 * m], scb = (float)(int8_t)b[192 + 8 * n + 2 * m + 1];
      const float pa = sca * sa, pb = scb * sb;
      return half_at(b, 208) * (pa + pb);
    }
  }
}

// twin/mod.rs:15-25 (tree): p[i] += p[i + s] for s = n/2, n/4, ..., 1; the result is p[0].
float tree(float* p, int n) {
  for (int s = n / 2; s > 0; s /= 2)
    for (int i = 0; i < s; ++i) p[i] = p[i] + p[i + s];
  return p[0];
}

}  // namespace

extern "C" {

// twin/matvec.rs:86-97 (row_dot) and 126-131 (matvec): lane l of 32 sums units l, l + 32, ... in
// order from 0, then the 32 partials meet in the tree.
int oc_matvec(uint32_t wtype, const uint8_t* w, uint64_t rows, uint64_t k, const float* x, float* y) {
  const uint64_t rb = oc_row_bytes(wtype, k);
  if (k % 32 != 0 || (rb == 0 && k != 0)) return 1;
  const uint64_t units = k / 32;
  for (uint64_t r = 0; r < rows; ++r) {
    float p[32];
    for (uint64_t lane = 0; lane < 32; ++lane) {
      float s = 0.0f;
      for (uint64_t u = lane; u < units; u += 32) s = s + unit_dot(wtype, w + r * rb, u, x);
      p[lane] = s;
    }
    y[r] = tree(p, 32);
  }
  return 0;
}


uint64_t oc_row_bytes(uint32_t wtype, uint64_t n) {
  if (wtype > 5 || n % kPer[wtype] != 0) return 0;
  return n / kPer[wtype] * kBytes[wtype];
}

int oc_dequant_row(uint32_t wtype, const uint8_t* row, uint64_t n, float* out) {
  if (oc_row_bytes(wtype, n) == 0 && n != 0) return 1;
  const uint64_t blocks = n / kPer[wtype];
  for (uint64_t k = 0; k < blocks; ++k) {
    const uint8_t* b = row + k * kBytes[wtype];
    float* o = out + k * kPer[wtype];
    switch (wtype) {
      case 0: std::memcpy(o, b, 4); break;
      case 1: {
        const uint32_t bits = (uint32_t)(b[0] | (b[1] << 8)) << 16;
        std::memcpy(o, &bits, 4);
        break;
      }
      case 2: q8_0_block(b, o); break;
      case 3: k4_block(b, nullptr, b + 16, o); break;
      case 4: k4_block(b, b + 16, b + 48, o); break;
      default: q6k_block(b, o); break;
    }
  }
  return 0;
}

float oc_half_to_float(uint16_t h) { return half_to_float(h); }

}  // extern "C"
