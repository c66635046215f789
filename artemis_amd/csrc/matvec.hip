// The output head's matvec, with the greedy draft step fused into it.
//
// matvec (crates/kernels/shaders/matvec.glsl, matvec_{type}.comp; dispatch Kernels::matvec):
// y = W x for `rows` rows of k values of a weight type (quant.glsl's six), each output as the
// reference computes it, bit for bit: lane l of a 32-lane row group sums the row's 32-value units
// l, l + 32, ... in order from 0 (quant.glsl's lane_sum; each unit_dot adds its rounded products in
// order), and the 32 partials meet in the tree p[i] += p[i + s] for s = 16, 8, 4, 2, 1
// (tree32.glsl; twin/mod.rs:15-25). The library is built without contraction, so every product is
// rounded before its add, as the reference's `precise` arithmetic is.
//
// On CDNA4 a wave of 64 lanes holds two 32-lane row groups (a 32-lane xor shuffle stays inside its
// half); each group computes two rows per step, so that two units' loads are in flight per lane,
// and a 256-thread workgroup walks 16-row steps grid-stride,
// with a grid that fits the chip in one round. x is staged once per workgroup in LDS, unit u at
// xs[33 u ..] (the pad of one float puts the 32 lanes' reads of 32 different units in 32 different
// banks). Weights are read once, straight from HBM; the compiler merges a unit's 2-byte reads into
// 16-byte loads (the target allows unaligned global access, and Q8_0 and Q6_K blocks, 34 and 210
// bytes, are only 2-byte aligned).
//
// head_argmax: the same rows with argmax_rows' epilogue (crates/kernels/shaders/argmax_rows.comp):
// the largest finite output, ties to the lower index (-0 and +0 tie), computed as the outputs are
// produced: each workgroup keeps its best as one u64 key, and a one-workgroup kernel takes the
// largest key and writes ids[slot] and rows_out[slot] = embd + id * row_bytes (AS_NO_DRAFT and row
// 0's address when no output is finite). The logits need not be written or read again.
#include "sampler_device.h"
#include "launch.h"
#include "../../include/artemis_sampler.h"

using namespace as_dev;

namespace {

constexpr uint32_t kThreads = 256;
constexpr uint32_t kRowsPerStep = 2 * (kThreads / 32);  // 8 groups of 32 lanes, two rows each
constexpr uint32_t kFinalThreads = 1024;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float half_u16(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }
// 32 bytes at a 2-byte aligned address as 8 words (two 2-byte reads each; the compiler merges the
// reads into wide loads), and byte l of them.
__device__ __forceinline__ void load32(const uint16_t* p, uint32_t (&q)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) q[i] = (uint32_t)p[2 * i] | ((uint32_t)p[2 * i + 1] << 16);
}
__device__ __forceinline__ uint32_t byte_of(const uint32_t (&q)[8], uint32_t l) {
  return (q[l >> 2] >> (8 * (l & 3))) & 0xFFu;
}

// quant.glsl unit_dot (twin/matvec.rs:21-84) for unit u of the row; x: the unit's 32 inputs in LDS.
template <uint32_t kType>
__device__ __forceinline__ float unit_dot(const uint8_t* __restrict__ row, uint32_t u, const float* x) {
  if constexpr (kType == AS_WTYPE_F32) {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(row + 128u * u);
    uint32_t wv[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) wv[i] = w[i];
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) s = s + __uint_as_float(wv[i]) * x[i];
    return s;
  } else if constexpr (kType == AS_WTYPE_BF16) {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(row + 64u * u);
    uint32_t wv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) wv[i] = w[i];
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s = s + __uint_as_float(wv[i] << 16) * x[2 * i];
      s = s + __uint_as_float(wv[i] & 0xFFFF0000u) * x[2 * i + 1];
    }
    return s;
  } else if constexpr (kType == AS_WTYPE_Q8_0) {
    const uint16_t* b = reinterpret_cast<const uint16_t*>(row + 34u * u);
    uint32_t q[8];
    load32(b + 1, q);
    const float d = half_u16(b[0]);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) s = s + (float)(int8_t)byte_of(q, i) * x[i];
    return d * s;
  } else if constexpr (kType == AS_WTYPE_Q4_K || kType == AS_WTYPE_Q5_K) {
    constexpr bool kQ5 = kType == AS_WTYPE_Q5_K;
    const uint8_t* blk = row + (kQ5 ? 176u : 144u) * (u / 8);
    const uint16_t* b = reinterpret_cast<const uint16_t*>(blk);
    const uint32_t j = u % 8, c = j / 2, sh = 4 * (j % 2);
    uint32_t hd[8], qs[8], qh[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) hd[i] = b[i];  // d, dmin, 12 bytes of scales and mins
    load32(b + (kQ5 ? 24 : 8) + 16 * c, qs);
    if constexpr (kQ5) load32(b + 8, qh);
    // ggml's get_scale_min_k4 over the 12 bytes at offset 4 (quant.glsl scale_min_k4).
    auto sb = [&](uint32_t i) { return (hd[2 + (i >> 1)] >> (8 * (i & 1))) & 0xFFu; };
    uint32_t sc, mn;
    if (j < 4) {
      sc = sb(j) & 63u;
      mn = sb(j + 4) & 63u;
    } else {
      sc = (sb(j + 4) & 0xFu) | ((sb(j - 4) >> 6) << 4);
      mn = (sb(j + 4) >> 4) | ((sb(j) >> 6) << 4);
    }
    float sq = 0.0f, sx = 0.0f;
    // Four quants at once, one a byte (quant.glsl kq_dot): the nibbles at sh and, for Q5_K, bit j of
    // the high bytes at bit 4; float(q) is exact, so the products are the reference's.
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t q4 = (qs[i] >> sh) & 0x0F0F0F0Fu;
      if constexpr (kQ5) q4 |= ((qh[i] >> j) & 0x01010101u) << 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sq = sq + (float)((q4 >> (8 * e)) & 0xFFu) * x[4 * i + e];
        sx = sx + x[4 * i + e];
      }
    }
    const float a = (half_u16(hd[0]) * (float)sc) * sq;
    const float m = (half_u16(hd[1]) * (float)mn) * sx;
    return a - m;
  } else {
    // Q6_K: unit j of a block is half n = j / 4, quarter m = j % 4.
    const uint16_t* b = reinterpret_cast<const uint16_t*>(row + 210u * (u / 8));
    const uint32_t j = u % 8, n = j / 4, m = j % 4;
    uint32_t ql[8], qh[8];
    load32(b + 32 * n + 16 * (m & 1), ql);
    load32(b + 64 + 16 * n, qh);
    const uint32_t scs = b[96 + 4 * n + m], dh = b[104];
    const uint32_t shl = 4 * (m >> 1), shh = 2 * m;
    float sa = 0.0f, sbs = 0.0f;
    // Four 6-bit quants q = lo + 16 hi at once, one a byte (the nibbles at shl, the 2-bit pairs at
    // shh), each byte holding q - 32 as a signed byte: lo in its low nibble and hi - 2 (mod 16) in its
    // high one, which v_perm_b32 looks up per byte (byte hi of 0x1000F0E0: 0xE0, 0xF0, 0x00, 0x10).
    // Each value is then one sign-extending byte-to-float conversion; float(q - 32) is exactly the
    // reference's float(q) - 32, so the products are its.
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t hi = __builtin_amdgcn_perm(0u, 0x1000F0E0u, (qh[i] >> shh) & 0x03030303u);
      const uint32_t s4 = ((ql[i] >> shl) & 0x0F0F0F0Fu) | hi;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float prod = (float)(int8_t)(uint8_t)(s4 >> (8 * e)) * x[4 * i + e];
        if (i < 4) sa = sa + prod;
        else sbs = sbs + prod;
      }
    }
    const float sca = (float)(int8_t)(scs & 0xFFu), scb = (float)(int8_t)(scs >> 8);
    const float pa = sca * sa, pb = scb * sbs;
    return half_u16(dh) * (pa + pb);
  }
}

// argmax_rows' order as one u64: finite values by value (-0 as +0), then the lower index; 0 for a
// non-finite value (below every finite key).
__device__ __forceinline__ uint64_t draft_key(float v, uint32_t i) {
  return is_finite_bits(v) ? pack(total_key(v == 0.0f ? 0.0f : v), i) : 0ull;
}

// Lane l's partials of two rows a and b: units l, l + 32, ... added in order from 0 (quant.glsl
// lane_sum). The two rows' dot products of a unit are independent and read the same inputs, so their
// loads are in flight together.
template <uint32_t kType>
__device__ __forceinline__ float lane_sum2(const uint8_t* wr, uint32_t lane, uint32_t units, const float* xs,
                                           float* acc_b, const uint8_t* wr_b, bool has_b) {
  float a = 0.0f, b = 0.0f;
  for (uint32_t u = lane; u < units; u += 32) {
    const float da = unit_dot<kType>(wr, u, xs + u * 33);
    const float db = has_b ? unit_dot<kType>(wr_b, u, xs + u * 33) : 0.0f;
    a = a + da;
    b = b + db;
  }
  *acc_b = b;
  return a;
}

// tree32.glsl over a 32-lane group (lanes past a short row's units hold +0.0).
__device__ __forceinline__ float tree32(float acc) {
  acc = acc + __shfl_xor(acc, 16, 32);
  acc = acc + __shfl_xor(acc, 8, 32);
  acc = acc + __shfl_xor(acc, 4, 32);
  acc = acc + __shfl_xor(acc, 2, 32);
  acc = acc + __shfl_xor(acc, 1, 32);
  return acc;
}

// Each 32-lane group computes two rows per step (a workgroup 16), rows 2s and 2s + 1 of the step.
template <uint32_t kType, bool kArgmax>
__global__ __launch_bounds__(kThreads) void matvec_kernel(const uint8_t* __restrict__ w, uint64_t row_bytes,
                                                          uint32_t rows, uint32_t k, const float* __restrict__ x,
                                                          float* __restrict__ y, uint64_t* __restrict__ partials) {
  extern __shared__ float xs[];  // k / 32 units of 33 floats
  __shared__ uint64_t red[kThreads / kWave];
  const uint32_t tid = threadIdx.x, units = k / 32;
  for (uint32_t i = tid; i < k; i += kThreads) xs[(i / 32) * 33 + (i % 32)] = x[i];
  __syncthreads();
  const uint32_t lane = tid & 31, slot = tid / 32;
  const uint32_t n_steps = (rows + kRowsPerStep - 1) / kRowsPerStep;
  uint64_t best = 0;
  for (uint32_t g = blockIdx.x; g < n_steps; g += gridDim.x) {
    const uint32_t r0 = g * kRowsPerStep + 2 * slot, r1 = r0 + 1;
    float acc0 = 0.0f, acc1 = 0.0f;
    if (r0 < rows)
      acc0 = lane_sum2<kType>(w + (uint64_t)r0 * row_bytes, lane, units, xs, &acc1, w + (uint64_t)r1 * row_bytes,
                              r1 < rows);
    acc0 = tree32(acc0);
    acc1 = tree32(acc1);
    if (lane == 0) {
      if (r0 < rows) {
        if (y) y[r0] = acc0;
        if (kArgmax) best = max(best, draft_key(acc0, r0));
      }
      if (r1 < rows) {
        if (y) y[r1] = acc1;
        if (kArgmax) best = max(best, draft_key(acc1, r1));
      }
    }
  }
  if constexpr (kArgmax) {
    best = wave_max_u64(best);
    if ((tid & (kWave - 1)) == 0) red[tid / kWave] = best;
    __syncthreads();
    if (tid == 0) {
      for (uint32_t i = 1; i < kThreads / kWave; ++i) best = max(best, red[i]);
      partials[blockIdx.x] = best;
    }
  }
}

__global__ __launch_bounds__(kFinalThreads) void draft_final_kernel(const uint64_t* __restrict__ partials,
                                                                    uint32_t n_partials, uint32_t* __restrict__ ids,
                                                                    uint64_t* __restrict__ rows_out, uint64_t embd,
                                                                    uint32_t row_bytes, uint32_t slot) {
  __shared__ uint64_t red[kFinalThreads / kWave];
  uint64_t best = 0;
  for (uint32_t i = threadIdx.x; i < n_partials; i += kFinalThreads) best = max(best, partials[i]);
  best = wave_max_u64(best);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (uint32_t i = 1; i < kFinalThreads / kWave; ++i) best = max(best, red[i]);
    const uint32_t id = best ? packed_id(best) : AS_NO_DRAFT;
    ids[slot] = id;
    rows_out[slot] = embd + (uint64_t)(best ? id : 0u) * (uint64_t)row_bytes;
  }
}

// Workgroups for `rows`: as many as the chip holds at once (the kernel's occupancy at this LDS size
// times the CUs), so every workgroup runs in the first round, and no more than there are steps.
template <typename K>
uint32_t grid_for(K kernel, size_t lds, uint32_t rows) {
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kThreads, lds) != hipSuccess || per_cu < 1 || cus < 1)
    per_cu = 1, cus = 256;
  uint64_t g = (uint64_t)per_cu * (uint64_t)cus;
  const uint32_t n_steps = (rows + kRowsPerStep - 1) / kRowsPerStep;
  if (g > as_launch::kMatvecGroups) g = as_launch::kMatvecGroups;
  return (uint32_t)(g < n_steps ? g : n_steps);
}

template <bool kArgmax>
hipError_t launch(hipStream_t stream, const void* w, uint32_t wtype, uint64_t row_bytes, uint32_t rows, uint32_t k,
                  const float* x, float* y, uint64_t* partials, uint32_t* groups) {
  const size_t lds = (size_t)(k / 32) * 33 * sizeof(float);
  const uint8_t* wb = static_cast<const uint8_t*>(w);
  const dim3 block(kThreads);
  switch (wtype) {
#define AS_MV(T)                                                                                                     \
  case T: {                                                                                                          \
    *groups = grid_for(matvec_kernel<T, kArgmax>, lds, rows);                                                        \
    hipLaunchKernelGGL((matvec_kernel<T, kArgmax>), dim3(*groups), block, lds, stream, wb, row_bytes, rows, k, x, y, \
                       partials);                                                                                    \
    break;                                                                                                           \
  }
    AS_MV(AS_WTYPE_F32)
    AS_MV(AS_WTYPE_BF16)
    AS_MV(AS_WTYPE_Q8_0)
    AS_MV(AS_WTYPE_Q4_K)
    AS_MV(AS_WTYPE_Q5_K)
    AS_MV(AS_WTYPE_Q6_K)
#undef AS_MV
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

namespace as_launch {

hipError_t matvec(hipStream_t stream, const void* w, uint32_t wtype, uint64_t row_bytes, uint32_t rows, uint32_t k,
                  const float* x, float* y) {
  uint32_t groups = 0;
  return launch<false>(stream, w, wtype, row_bytes, rows, k, x, y, nullptr, &groups);
}

hipError_t head_argmax(hipStream_t stream, const void* w, uint32_t wtype, uint64_t row_bytes, uint32_t rows,
                       uint32_t k, const float* x, float* y, uint64_t* partials, uint32_t* ids, uint64_t* rows_out,
                       uint64_t embd, uint32_t embd_row_bytes, uint32_t slot) {
  uint32_t groups = 0;
  hipError_t e = launch<true>(stream, w, wtype, row_bytes, rows, k, x, y, partials, &groups);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(draft_final_kernel, dim3(1), dim3(kFinalThreads), 0, stream, partials, groups, ids, rows_out,
                     embd, embd_row_bytes, slot);
  return hipGetLastError();
}

}  // namespace as_launch
