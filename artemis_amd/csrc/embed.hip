// embed_rows: the draft chain's second step (crates/kernels/src/dispatch.rs:97-120,
// shaders/embed_rows.comp). For each token t, y[t][0..n) is the embedding row at address rows[t]
// dequantized as qwen36::quant::dequant_row does (crates/qwen36/src/quant.rs:77-252): ggml's block
// layouts for F32, BF16, Q8_0, Q4_K, Q5_K and Q6_K, each value from the same f32 operations in the
// same order (products rounded before the subtraction: the library is built without contraction),
// so the output is the reference's bit for bit.
//
// The addresses come from argmax_rows (rows[slot] = embd + id * row_bytes), so the chain
// logits -> draft id -> embedding runs on the GPU without a host round trip. On MI355X the table
// lives in HBM (288 GB holds any embedding table of the family); a pinned host table works too.
//
// One 256-thread workgroup per (256-value group, token). A group starts on a block boundary for
// every type (Q8_0's 32-value blocks divide 256; the K-quants' blocks are 256 values), so the
// quantized types stage the group's bytes (at most 272) into LDS with 2-byte loads (Q8_0 and Q6_K
// blocks, 34 and 210 bytes, are only 2-byte aligned) and each thread decodes its value from LDS.
// Every address must be 2-byte aligned (each row of a 2-byte aligned table is: every row size is
// even); an odd one gives NaN for its row instead of a load.
#include "sampler_device.h"
#include "launch.h"
#include "../../include/artemis_sampler.h"

namespace {

constexpr uint32_t kGroup = 256;
constexpr uint32_t kStage = 272;  // bytes of the largest quantized group (8 Q8_0 blocks)

__device__ __forceinline__ float half_bits(uint32_t lo, uint32_t hi) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(lo | (hi << 8)));
}

// quant.rs:170-179 (ggml's get_scale_min_k4): scale and min of sub-block j from 12 packed bytes.
__device__ __forceinline__ void scale_min_k4(uint32_t j, const uint8_t* q, uint32_t* sc, uint32_t* m) {
  if (j < 4) {
    *sc = q[j] & 63u;
    *m = q[j + 4] & 63u;
  } else {
    *sc = (q[j + 4] & 0xFu) | ((uint32_t)(q[j - 4] >> 6) << 4);
    *m = (uint32_t)(q[j + 4] >> 4) | ((uint32_t)(q[j] >> 6) << 4);
  }
}

template <uint32_t kType>
__global__ __launch_bounds__(kGroup) void embed_rows_kernel(const uint64_t* __restrict__ rows, uint32_t n,
                                                            float* __restrict__ y) {
  __shared__ uint16_t stage[kStage / 2];
  const uint32_t g = blockIdx.x, t = blockIdx.y, e = threadIdx.x;
  const uint64_t addr = rows[t];
  const uint32_t i = g * kGroup + e;
  float* out = y + (uint64_t)t * n;
  if (addr & 1u) {
    if (i < n) out[i] = __builtin_nanf("");
    return;
  }
  const uint16_t* row = reinterpret_cast<const uint16_t*>(addr);

  if constexpr (kType == AS_WTYPE_F32) {
    if (i < n) out[i] = __uint_as_float((uint32_t)row[2 * i] | ((uint32_t)row[2 * i + 1] << 16));
    return;
  } else if constexpr (kType == AS_WTYPE_BF16) {
    if (i < n) out[i] = __uint_as_float((uint32_t)row[i] << 16);  // quant.rs:86-89
    return;
  } else {
    // The group's bytes into LDS: whole blocks of the group that lie in the row.
    constexpr uint32_t kPer = kType == AS_WTYPE_Q8_0 ? 32u : 256u;
    constexpr uint32_t kBytes = kType == AS_WTYPE_Q8_0 ? 34u : kType == AS_WTYPE_Q4_K ? 144u
                                : kType == AS_WTYPE_Q5_K ? 176u : 210u;
    const uint32_t vals = min(kGroup, n - g * kGroup);
    const uint32_t words = vals / kPer * kBytes / 2;
    const uint16_t* src = row + (uint64_t)g * (kGroup / kPer) * kBytes / 2;
    for (uint32_t w = e; w < words; w += kGroup) stage[w] = src[w];
    __syncthreads();
    if (i >= n) return;
    const uint8_t* b = reinterpret_cast<const uint8_t*>(stage);
    float v;
    if constexpr (kType == AS_WTYPE_Q8_0) {
      // quant.rs:161-167: d * q.
      const uint8_t* blk = b + (e / 32) * 34;
      v = half_bits(blk[0], blk[1]) * (float)(int8_t)blk[2 + e % 32];
    } else if constexpr (kType == AS_WTYPE_Q4_K || kType == AS_WTYPE_Q5_K) {
      // quant.rs:182-228: value l of sub-block j = 2c + hi is (d * scale_j) * q - dmin * min_j.
      const uint32_t c = e / 64, hi = (e % 64) / 32, l = e % 32, j = 2 * c + hi;
      uint32_t sc, mn;
      scale_min_k4(j, b + 4, &sc, &mn);
      const float d1 = half_bits(b[0], b[1]) * (float)sc;
      const float mm = half_bits(b[2], b[3]) * (float)mn;
      uint32_t q = (b[(kType == AS_WTYPE_Q4_K ? 16u : 48u) + 32 * c + l] >> (4 * hi)) & 0xFu;
      if (kType == AS_WTYPE_Q5_K && ((b[16 + l] >> j) & 1u)) q += 16u;
      const float p = d1 * (float)q;
      v = p - mm;
    } else {
      // quant.rs:231-252: half h, quarter m, lane l: (d * scale) * (6-bit q - 32).
      const uint32_t h = e / 128, m = (e % 128) / 32, l = e % 32;
      const uint32_t lo = (b[64 * h + 32 * (m & 1) + l] >> (4 * (m >> 1))) & 0xFu;
      const uint32_t hb = (b[128 + 32 * h + l] >> (2 * m)) & 3u;
      const float s = half_bits(b[208], b[209]) * (float)(int8_t)b[192 + 8 * h + 2 * m + l / 16];
      v = s * (float)((int)(lo | (hb << 4)) - 32);
    }
    out[i] = v;
  }
}

}  // namespace

namespace as_launch {

hipError_t embed_rows(hipStream_t stream, const uint64_t* rows, uint32_t wtype, uint32_t n, float* y,
                      uint32_t n_tokens) {
  const dim3 grid((n + kGroup - 1) / kGroup, n_tokens);
  switch (wtype) {
    case AS_WTYPE_F32: hipLaunchKernelGGL(embed_rows_kernel<AS_WTYPE_F32>, grid, dim3(kGroup), 0, stream, rows, n, y); break;
    case AS_WTYPE_BF16: hipLaunchKernelGGL(embed_rows_kernel<AS_WTYPE_BF16>, grid, dim3(kGroup), 0, stream, rows, n, y); break;
    case AS_WTYPE_Q8_0: hipLaunchKernelGGL(embed_rows_kernel<AS_WTYPE_Q8_0>, grid, dim3(kGroup), 0, stream, rows, n, y); break;
    case AS_WTYPE_Q4_K: hipLaunchKernelGGL(embed_rows_kernel<AS_WTYPE_Q4_K>, grid, dim3(kGroup), 0, stream, rows, n, y); break;
    case AS_WTYPE_Q5_K: hipLaunchKernelGGL(embed_rows_kernel<AS_WTYPE_Q5_K>, grid, dim3(kGroup), 0, stream, rows, n, y); break;
    case AS_WTYPE_Q6_K: hipLaunchKernelGGL(embed_rows_kernel<AS_WTYPE_Q6_K>, grid, dim3(kGroup), 0, stream, rows, n, y); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace as_launch
