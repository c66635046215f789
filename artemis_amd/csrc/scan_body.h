// The scan's body: pass 1 over the logits, one slice of one row per workgroup (see scan.hip for the
// algorithm). Included by a kernel file after it defines
//   AS_SCAN_NS         the namespace of this copy,
//   AS_SCAN_THREADS    threads per workgroup (a multiple of 64),
//   AS_SCAN_HASH       LDS hash slots for the slice's distinct history ids (a multiple of the threads),
//   AS_SCAN_SLICE_MAX  the longest slice (its history bitmap lives in LDS),
//   AS_SCAN_DEPTH      chunk buffers per wave (the loads of all but one are in flight),
// The entry point is AS_SCAN_NS::scan_slice.
namespace {
namespace AS_SCAN_NS {

using namespace as_dev;

constexpr int kThreads = AS_SCAN_THREADS;
constexpr int kWaves = kThreads / kWave;
constexpr int kU = 4;                           // 16-byte loads per lane per chunk
constexpr int kDepth = AS_SCAN_DEPTH;           // chunk buffers per wave (kDepth - 1 in flight)
static_assert(kDepth >= 2, "a chunk in flight while one is worked on");
constexpr uint32_t kChunk = kWave * 4 * kU;     // values per wave chunk (1,024)
constexpr uint32_t kGroupStep = kWaves * kChunk;
constexpr uint32_t kCapW = as_launch::kWaveCap;
constexpr int kQ = kCapW / kWave;               // buffer entries per lane when a wave reads it whole
constexpr uint32_t kRoom = 4 * kWave;           // the most one 16-byte group per lane appends
// Rows without a top-k start from the 16th best of each wave's first chunk: shared over a row's
// waves, about its 2,000th-3,000th value, near the depth their selects keep, so that few run.
constexpr uint32_t kFirstRankPartial = 16;
// Waves read the row's shared words once per kShareEvery chunks (an even number): the read is an
// agent-scope load, slower than the stream's own, and loads complete in order, so each read delays
// the chunk loaded after it (measured: every two chunks cost ~7 us per top-k slice over every eight).
constexpr uint32_t kShareEvery = 8;
static_assert(kShareEvery % 2 == 0, "reads fall on the loop's odd chunks");
constexpr uint32_t kHash = AS_SCAN_HASH;
constexpr int kHashPer = (kHash + kThreads - 1) / kThreads;  // hash slots per thread (the last may be short)
constexpr int kHxEarly = 2;  // slots per thread whose raw values load before the stream
// The table's first kHashPrimary slots are those of each thread's first kHxEarly (raw values loaded
// before the stream): a short history's ids all go there.
constexpr uint32_t kHashPrimary = (uint32_t)kThreads * 2u < kHash ? (uint32_t)kThreads * 2u : kHash;
constexpr int kPrimaryShift = 32 - __builtin_ctz(kHashPrimary);  // the multiplicative hash's top bits
constexpr uint32_t kPrimaryProbes = 16;
static_assert((kHashPrimary & (kHashPrimary - 1)) == 0 && kHashPrimary < kHash, "a power-of-two first part");
static_assert((kHash & (kHash - 1)) == 0, "a power of two");
constexpr uint32_t kEmpty = 0xFFFFFFFFu;
typedef float f32x4 __attribute__((ext_vector_type(4)));
static_assert(kCapW % kWave == 0, "sizes");
// Thread tid holds hash slots tid + k * kThreads, k < kHashPer, those below kHash.
__device__ __forceinline__ bool own_slot(uint32_t tid, int k) { return kHash % kThreads == 0 || tid + k * kThreads < kHash; }
static_assert(as_launch::kSliceAlign % kChunk == 0, "slices start on a chunk");
static_assert(as_launch::kTopKMax + as_launch::kTopKMax / 4 + kRoom <= kCapW &&
                  as_launch::kFloorRank + as_launch::kFloorRank / 4 + kRoom <= kCapW,
              "a select always leaves room for one group");

// What a slice computes besides the non-finite check.
enum Kind : int {
  kKindPlain = 0,      // greedy rows (and rows the finish kernel settles on its own)
  kKindCand = 1,       // candidates (with min-p's floor when the row has one)
  kKindSumTop = 2,     // candidates and sums of exp(l - m)
  kKindSumTemp = 3,    // candidates and sums of exp((l - m) / T)
};

struct Shared {
  uint64_t buf[kWaves][kCapW];
  uint32_t bitmap[AS_SCAN_SLICE_MAX / 32];
  uint32_t hid[kHash];
  uint32_t hcnt[kHash];
  uint64_t red_p[kWaves];
  uint32_t red_u[kWaves];
  uint32_t red_u2[kWaves];
  uint32_t red_u3[kWaves];
  float red_f[kWaves];
  double red_d[kWaves];
  double red_d2[kWaves];
  uint32_t hist_out;
  uint32_t overflow;
  uint32_t out_n;  // candidates the waves have written to HBM during the stream
  uint32_t vast;   // a wave found min-p's floor set vast (two in five of its first chunk)
  RowParams prm;   // the row's parameters
};
// The workgroup's LDS, at file scope so that the out-of-line helpers below address it directly.
__shared__ Shared g_sh_static;
__device__ __forceinline__ Shared& shm() { return g_sh_static; }

__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t u = __shfl_xor(v, o, kWave);
    v = u < v ? u : v;
  }
  return v;
}

// The row's shared words (RowShare::bound, top, the slots) live in device memory and are accessed at
// agent scope: a row's slices run on different XCDs.
constexpr int kShareScope = __HIP_MEMORY_SCOPE_AGENT;
__device__ __forceinline__ void publish(uint32_t* word, uint32_t key) {
  if (word && (threadIdx.x & (kWave - 1)) == 0) __hip_atomic_fetch_max(word, key, __ATOMIC_RELAXED, kShareScope);
}
__device__ __forceinline__ uint64_t read_shared(uint32_t* words) {
  return __hip_atomic_load(reinterpret_cast<uint64_t*>(words), __ATOMIC_RELAXED, kShareScope);
}

// A wave's candidate buffer (shm().buf[wave]): it holds every value of the wave's stream so far
// whose packed rank is >= tau (tau 0: every value), `cnt` entries, some of which may rank below tau.
// The same in every lane; passed and returned by value so that the out-of-line helpers keep it in
// registers.
struct WaveState {
  uint32_t cnt;
  float tau_f;   // the value of tau's key: a value below it cannot rank >= tau
  uint64_t tau;
  uint32_t top;  // min-p rows: the largest key the wave knows the row to hold (0: none yet)
  uint32_t C;    // the count a select keeps (at most C + C / 4 of them)
  uint32_t sel;  // the buffer count at which a chunk ends with a select
  bool spill;    // min-p rows keeping every value above the floor: a full buffer goes to HBM
};

// The state as scalars: it comes back from the out-of-line helpers in vector registers, and the
// stream's tests and counts on it are cheaper on scalar ones.
__device__ __forceinline__ WaveState uniform(WaveState ws) {
  ws.cnt = __builtin_amdgcn_readfirstlane(ws.cnt);
  ws.tau_f = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(uint32_t, ws.tau_f)));
  // (readfirstlane returns a signed int: each half goes through uint32_t before it widens)
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(ws.tau >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)ws.tau);
  ws.tau = ((uint64_t)hi << 32) | lo;
  ws.top = __builtin_amdgcn_readfirstlane(ws.top);
  ws.C = __builtin_amdgcn_readfirstlane(ws.C);
  ws.sel = __builtin_amdgcn_readfirstlane(ws.sel);
  ws.spill = __builtin_amdgcn_readfirstlane(ws.spill ? 1u : 0u) != 0u;
  return ws;
}

// Selects run once the buffer holds twice C (at least C + 64, at most all but one wave's worth of
// entries), and whenever a group's values would not fit.
__device__ __forceinline__ uint32_t select_at(uint32_t C) { return min(max(2 * C, C + 64), kCapW - kWave); }

__device__ __forceinline__ void raise_tau(WaveState& ws, uint64_t t) {
  if (t > ws.tau) {
    ws.tau = t;
    ws.tau_f = key_value((uint32_t)(t >> 32));
  }
}

// min-p's floor for a row whose largest value has key `top`: the smallest value that can be kept.
__device__ __forceinline__ uint64_t floor_tau(uint32_t top, double ln_min_p) {
  return (uint64_t)total_key(floor_f32((double)key_value(top) + ln_min_p)) << 32;
}

// A packed rank t with at least C and at most C + slack of the kN values per lane (0: none) at or
// above it, as high as that allows: by ballot counts on the key, halving the key range until the
// count at its low end is within the slack, then (slack 0, or heavy ties) among ties at that key on
// the low word. 0 when fewer than C values are given. Every given value's key must be >= lo.
template <int kN>
__device__ __forceinline__ uint64_t wave_kth(const uint64_t (&ent)[kN], uint32_t C, uint32_t lo, uint32_t slack) {
  uint32_t kmax = 0, total = 0;
#pragma unroll
  for (int q = 0; q < kN; ++q) {
    if (ent[q] != 0ull) kmax = max(kmax, (uint32_t)(ent[q] >> 32));
    total += (uint32_t)__popcll(__ballot(ent[q] != 0ull));
  }
  if (total < C || C == 0) return 0ull;
  if (total <= C + slack) return (uint64_t)lo << 32;
  kmax = wave_max_u32(kmax);
  uint64_t hi = (uint64_t)kmax + 1;  // count(key >= hi) = 0 < C; count(key >= lo) >= C
  uint32_t c_hi = 0;
  while (hi - lo > 1) {
    const uint32_t mid = (uint32_t)(lo + ((hi - lo) >> 1));
    uint32_t c = 0;
#pragma unroll
    for (int q = 0; q < kN; ++q) c += (uint32_t)__popcll(__ballot(ent[q] != 0ull && (uint32_t)(ent[q] >> 32) >= mid));
    if (c >= C) {
      lo = mid;
      if (c <= C + slack) return (uint64_t)lo << 32;
    } else {
      hi = mid;
      c_hi = c;
    }
  }
  uint32_t c_ge = 0;
#pragma unroll
  for (int q = 0; q < kN; ++q) c_ge += (uint32_t)__popcll(__ballot(ent[q] != 0ull && (uint32_t)(ent[q] >> 32) >= lo));
  if (c_ge <= C + slack && c_ge != C) return (uint64_t)lo << 32;
  if (c_ge == C) {
    uint64_t mn = ~0ull;
#pragma unroll
    for (int q = 0; q < kN; ++q)
      if (ent[q] != 0ull && (uint32_t)(ent[q] >> 32) >= lo && ent[q] < mn) mn = ent[q];
    return wave_min_u64(mn);
  }
  // c_hi < C < c_ge: the C - c_hi ties at lo with the largest low words (the lowest ids).
  const uint32_t need = C - c_hi;
  uint64_t l2 = 0, h2 = 1ull << 32;
  while (h2 - l2 > 1) {
    const uint32_t mid = (uint32_t)(l2 + ((h2 - l2) >> 1));
    uint32_t c = 0;
#pragma unroll
    for (int q = 0; q < kN; ++q)
      c += (uint32_t)__popcll(__ballot(ent[q] != 0ull && (uint32_t)(ent[q] >> 32) == lo && (uint32_t)ent[q] >= mid));
    if (c >= need) l2 = mid;
    else h2 = mid;
  }
  return ((uint64_t)lo << 32) | l2;
}

// Drops the entries below tau (which may have risen since they were appended) and, when more than
// C remain, keeps the best C to C + slack, raises tau to the last kept and publishes its key to the
// row (share null: not). Every value the wave streams later has a larger id than those held, so the
// buffer stays exactly the wave's values >= tau. kN: entries read per lane (cnt <= kN * 64). Out of
// line: it runs a few times a slice.
template <int kN>
__device__ __noinline__ WaveState wave_select(WaveState ws, uint32_t C, uint32_t slack, uint32_t* share) {
  const uint32_t lane = threadIdx.x & (kWave - 1);
  uint64_t* buf = shm().buf[threadIdx.x / kWave];
  uint64_t ent[kN];
  uint32_t n_ge = 0;
#pragma unroll
  for (int q = 0; q < kN; ++q) {
    const uint32_t i = lane + q * kWave;
    const uint64_t e = (i < ws.cnt) ? buf[i] : 0ull;
    ent[q] = e >= ws.tau ? e : 0ull;
    n_ge += (uint32_t)__popcll(__ballot(ent[q] != 0ull));
  }
  if (n_ge > C) {
    const uint64_t t = wave_kth<kN>(ent, C, (uint32_t)(ws.tau >> 32), slack);
    raise_tau(ws, t);
    publish(share, (uint32_t)(t >> 32));
  }
  uint32_t run = 0;
#pragma unroll
  for (int q = 0; q < kN; ++q) {
    const bool keep = ent[q] != 0ull && ent[q] >= ws.tau;
    const uint64_t m = __ballot(keep);
    if (keep) buf[run + lanes_below(m)] = ent[q];
    run += (uint32_t)__popcll(m);
  }
  ws.cnt = run;
  return ws;
}

__device__ __forceinline__ void select_now(WaveState& ws, uint32_t C, uint32_t slack, uint32_t* share) {
  if (ws.cnt <= 2 * kWave) ws = uniform(wave_select<2>(ws, C, slack, share));
  else if (ws.cnt <= 6 * kWave) ws = uniform(wave_select<6>(ws, C, slack, share));
  else ws = uniform(wave_select<kQ>(ws, C, slack, share));
  static_assert(kQ > 6, "three sizes");
}

// A min-p row's full buffer: the entries >= tau (the floor may have risen since they were appended)
// stay when they are at most C; otherwise they go to the slice's candidates in HBM, after those
// already there, and the buffer empties. When they would pass `room`, the floor set is too large to
// keep whole: the wave keeps its best kPartialRank from then on, like a row without min-p (the floor
// still applies). Out of line: it runs when a min-p row's buffer fills.
__device__ __noinline__ WaveState spill(WaveState ws, uint64_t* out, uint32_t room, uint32_t* share) {
  const uint32_t lane = threadIdx.x & (kWave - 1);
  uint64_t* buf = shm().buf[threadIdx.x / kWave];
  uint64_t ent[kQ];
  uint32_t n_ge = 0;
#pragma unroll
  for (int q = 0; q < kQ; ++q) {
    const uint32_t i = lane + q * kWave;
    const uint64_t e = (i < ws.cnt) ? buf[i] : 0ull;
    ent[q] = e >= ws.tau ? e : 0ull;
    n_ge += (uint32_t)__popcll(__ballot(ent[q] != 0ull));
  }
  if (n_ge <= ws.C) {
    uint32_t run = 0;
#pragma unroll
    for (int q = 0; q < kQ; ++q) {
      const bool keep = ent[q] != 0ull;
      const uint64_t m = __ballot(keep);
      if (keep) buf[run + lanes_below(m)] = ent[q];
      run += (uint32_t)__popcll(m);
    }
    ws.cnt = run;
    return ws;
  }
  uint32_t base = kNone;
  if (lane == 0) {
    uint32_t old = shm().out_n;
    while (old + n_ge <= room) {
      const uint32_t prev = atomicCAS(&shm().out_n, old, old + n_ge);
      if (prev == old) {
        base = old;
        break;
      }
      old = prev;
    }
  }
  base = __builtin_amdgcn_readfirstlane(base);
  if (base == kNone) {
    ws.spill = false;
    ws.C = as_launch::kPartialRank;
    ws.sel = select_at(ws.C);
    select_now(ws, ws.C, ws.C / 4, share);
    return ws;
  }
  uint32_t run = base;
#pragma unroll
  for (int q = 0; q < kQ; ++q) {
    const bool keep = ent[q] != 0ull;
    const uint64_t m = __ballot(keep);
    if (keep) out[run + lanes_below(m)] = ent[q];
    run += (uint32_t)__popcll(m);
  }
  ws.cnt = 0;
  return ws;
}

// The starting threshold from the wave's first chunk (16 values per lane, those with a bit set in
// `masked` left out): the lane's two best by rank, then the wave's C-th best of those 128, which at
// least C values of the chunk meet (with C above 128, the 128th); published to the row. Fewer valid
// values leave it at 0. Inline, as first_floor: it runs while the wave's next chunk is in flight,
// and an out-of-line call begins by waiting for every load the wave has issued.
__device__ __forceinline__ WaveState first_tau(WaveState ws, f32x4 v0, f32x4 v1, f32x4 v2, f32x4 v3,
                                            uint32_t masked, uint32_t e0, uint32_t C, uint32_t* share,
                                            uint32_t* slot, uint32_t q) {
  const f32x4 v[kU] = {v0, v1, v2, v3};
  uint64_t top[2] = {0ull, 0ull};
#pragma unroll
  for (int j = 0; j < kU; ++j) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if ((masked >> (4 * j + c)) & 1u || !is_finite_bits(v[j][c])) continue;
      const uint64_t pk = pack(total_key(v[j][c]), e0 + j * (kWave * 4) + c);
      if (pk > top[0]) {
        top[1] = top[0];
        top[0] = pk;
      } else if (pk > top[1]) {
        top[1] = pk;
      }
    }
  }
  const uint64_t t = wave_kth<2>(top, min(C, 2u * kWave), 0u, 0u);
  if (t != 0ull) {
    raise_tau(ws, t);
    publish(share, (uint32_t)(t >> 32));
  }
  if (slot) {
    const uint64_t tq = wave_kth<2>(top, q, 0u, 0u);
    if (tq != 0ull) publish(slot, (uint32_t)(tq >> 32));
  }
  return ws;
}

// The q-th largest of the lanes' x (0 when fewer than q lanes hold a nonzero x): at most q rounds
// of a wave maximum.
__device__ __forceinline__ uint32_t wave_qth(uint32_t x, uint32_t q) {
  uint32_t need = q;
  for (uint32_t it = 0; it < q; ++it) {
    const uint32_t m = wave_max_u32(x);
    if (m == 0) return 0;
    const uint32_t c = (uint32_t)__popcll(__ballot(x == m));
    if (c >= need) return m;
    need -= c;
    if (x == m) x = 0;
  }
  return 0;
}

// The largest unmasked value of the wave's first chunk sets min-p's first floor. When more than one
// in a hundred of the chunk's values pass it (a floor set of thousands, or a first chunk whose
// largest value lies far below the row's: appending and spilling each value above it would cost
// more than keeping the best few hundred), the wave keeps its best kPartialRank like a row without
// min-p instead of every value above the floor (which still applies). When two in five pass, the
// slice notes the floor set as vast (tens of thousands of values).
__device__ __forceinline__ WaveState first_floor(WaveState ws, f32x4 v0, f32x4 v1, f32x4 v2, f32x4 v3,
                                              uint32_t masked, uint32_t e0, double ln_min_p, uint32_t* share) {
  const f32x4 v[kU] = {v0, v1, v2, v3};
  uint32_t k = 0;
#pragma unroll
  for (int j = 0; j < kU; ++j)
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (!((masked >> (4 * j + c)) & 1u) && is_finite_bits(v[j][c])) k = max(k, total_key(v[j][c]));
  k = wave_max_u32(k);
  if (k > ws.top) {
    ws.top = k;
    publish(share + 1, k);
    raise_tau(ws, floor_tau(k, ln_min_p));
  }
  uint32_t n_f = 0, n_v = 0;
#pragma unroll
  for (int j = 0; j < kU; ++j)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bool valid = !((masked >> (4 * j + c)) & 1u);
      n_v += (uint32_t)__popcll(__ballot(valid));
      n_f += (uint32_t)__popcll(__ballot(valid && v[j][c] >= ws.tau_f));
    }
  if (100 * n_f > n_v && ws.spill) {
    ws.spill = false;
    // Past two in five, the floor set is tens of thousands: it cannot stay whole, and the wave keeps
    // the depth of a row without min-p.
    ws.C = as_launch::kPartialRank;
    if (5 * n_f > 2 * n_v && (threadIdx.x & (kWave - 1)) == 0) shm().vast = 1;
    ws.sel = select_at(ws.C);
    ws = first_tau(ws, v0, v1, v2, v3, masked, e0, kFirstRankPartial, share, nullptr, 0u);
  }
  return ws;
}

struct Slice {
  const float* x;       // the row
  const float* zero;    // kChunk readable zeros, for the loads of a wave with no full chunk
  uint32_t* share;      // the row's shared words
  uint32_t* slots;      // the row's slots (top-k rows), n_slots of them; mine (or null)
  uint32_t* my_slot;
  uint32_t n_slots;
  uint32_t q;           // the rank each slot holds
  uint32_t b0, b1;      // the slice's values [b0, b1)
  uint32_t C;           // candidates per wave
  uint64_t* out;        // the slice's candidates in HBM
  uint32_t room;        // how many of them the stream may write
  bool first;           // the first chunk sets tau, to its first_rank-th best
  uint32_t first_rank;
  bool pen;             // history values are left out of the stream
  bool floor_on;        // min-p's floor applies to the candidates (a row without a top-k)
  float scale;          // log2(e), or log2(e) / T for sums of exp((l - m) / T)
  double ln_min_p;
};

// The bits of values e0 .. e0+3 (e0 - b0 a multiple of 4, e0 < b1) in the slice's history bitmap.
__device__ __forceinline__ uint32_t hist_nibble(const Slice& sl, uint32_t e0) {
  const uint32_t off = e0 - sl.b0;
  return (shm().bitmap[off >> 5] >> (off & 31u)) & 15u;
}
// The values of a 16-byte group the stream leaves out: history ids and, in the tail, those past b1.
template <bool kTail>
__device__ __forceinline__ uint32_t group_mask(const Slice& sl, uint32_t e0) {
  uint32_t m = 0;
  if (sl.pen && (!kTail || e0 < sl.b1)) m = hist_nibble(sl, e0);
  if (kTail) {
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (e0 + c >= sl.b1) m |= 1u << c;
  }
  return m;
}

struct Lane {
  float nfa;        // fma(x, 0, nfa) over the raw values: NaN once one is NaN or infinite
  float gv;         // greedy
  uint32_t gi;
  uint32_t amax;    // the largest key this lane appended
  float ref;        // the lane's largest raw value so far (-inf before any)
  double s;         // sum of exp2(t), t = (l - ref) * scale
  float sa;         // sum of exp2(t) * |t|: an error-bound term, kept roughly
  uint32_t moves;   // times ref moved while s held terms
};

// Appends the values e0 .. e0+3 of one 16-byte group that reach tau's value and are not masked to
// the wave's buffer, first making room when the values reaching tau would not fit. A value's test
// is one compare; the mask is looked at only when some lane passes it.
__device__ __forceinline__ void append4(WaveState& ws, Lane& ln, const f32x4& v, uint32_t e0, uint32_t mask,
                                        const Slice& sl) {
  if (ws.cnt > kCapW - kRoom) {
    uint32_t need = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) need += (uint32_t)__popcll(__ballot(v[c] >= ws.tau_f));
    if (ws.cnt + need > kCapW) {
      if (ws.spill) ws = uniform(spill(ws, sl.out, sl.room, sl.share));
      else select_now(ws, ws.C, ws.C / 4, sl.share);
    }
  }
  uint64_t* buf = shm().buf[__builtin_amdgcn_readfirstlane(threadIdx.x / kWave)];
  const uint32_t nid = ~e0;  // e0 + c packs as nid - c
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    if (__ballot(v[c] >= ws.tau_f) == 0ull) continue;
    const bool take = v[c] >= ws.tau_f && !((mask >> c) & 1u);
    const uint64_t m = __ballot(take);
    if (take) {
      const uint32_t key = total_key(v[c]);
      buf[ws.cnt + lanes_below(m)] = ((uint64_t)key << 32) | (nid - c);
      ln.amax = max(ln.amax, key);
    }
    ws.cnt += (uint32_t)__popcll(m);
  }
}

// exp2 through the hardware (V_EXP_F32). Its error is bounded per term by the callers: the
// instruction's own (kExpUlp units of 2^-23), plus at most 4 * 2^-24 * |t| for the roundings of t
// (the difference, the rounded scale and the product).
constexpr float kLog2e = 1.44269502f;
constexpr float kExpUlp = 2.0f;

// Moves the lane's reference up to m (> ref): the sums are rescaled by exp2(-dt) and every |t| they
// hold grows by dt.
__device__ __forceinline__ void move_ref(Lane& ln, float m, float scale) {
  if (ln.s != 0.0) {
    const float dt = (m - ln.ref) * scale;
    const float sc = __builtin_amdgcn_exp2f(-dt);
    ln.sa = sc * fmaf((float)ln.s, dt, ln.sa);
    ln.s = ln.s * (double)sc;
    ++ln.moves;
  }
  ln.ref = m;
}

// One wave chunk: kU 16-byte groups per lane, group j of lane l at e = c0 + j*256 + l*4. kFirst: the
// wave's first chunk, which sets the starting threshold.
template <int kKind, bool kTail, bool kFirst>
__device__ __forceinline__ void chunk(Lane& ln, WaveState& ws, const Slice& sl,
                                      const f32x4 (&q)[kU], uint32_t c0) {
  const uint32_t lane = threadIdx.x & (kWave - 1);
  constexpr bool kSums = kKind == kKindSumTop || kKind == kKindSumTemp;
#pragma unroll
  for (int j = 0; j < kU; ++j)
#pragma unroll
    for (int c = 0; c < 4; ++c) ln.nfa = fmaf(q[j][c], 0.0f, ln.nfa);

  if (kKind == kKindPlain) {
    float cm = q[0][0];
#pragma unroll
    for (int j = 0; j < kU; ++j)
#pragma unroll
      for (int c = 0; c < 4; ++c) cm = fmaxf(cm, q[j][c]);
    if (cm > ln.gv || ln.gi == kNone || kTail) {
#pragma unroll
      for (int j = 0; j < kU; ++j) {
        const uint32_t e0 = c0 + j * (kWave * 4) + lane * 4;
        const uint32_t m = group_mask<kTail>(sl, e0);
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (!((m >> c) & 1u) && (q[j][c] > ln.gv || ln.gi == kNone)) {
            ln.gv = q[j][c];
            ln.gi = e0 + c;
          }
      }
    }
    return;
  }

  constexpr bool kMasks = kFirst || kSums || kTail;
  uint32_t mask[kU];
#pragma unroll
  for (int j = 0; j < kU; ++j) mask[j] = kMasks ? group_mask<kTail>(sl, c0 + j * (kWave * 4) + lane * 4) : 0u;

  if (kFirst) {
    const uint32_t all = mask[0] | mask[1] << 4 | mask[2] << 8 | mask[3] << 12;
    if (sl.floor_on) ws = uniform(first_floor(ws, q[0], q[1], q[2], q[3], all, c0 + lane * 4, sl.ln_min_p, sl.share));
    else if (sl.first) ws = uniform(first_tau(ws, q[0], q[1], q[2], q[3], all, c0 + lane * 4, sl.first_rank, sl.share, sl.my_slot, sl.q));
  }
  float m4[kU];
#pragma unroll
  for (int j = 0; j < kU; ++j) {
    const f32x4 v = q[j];
    m4[j] = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
    if (__builtin_expect(__ballot(m4[j] >= ws.tau_f) != 0ull, 0)) {
      const uint32_t e0 = c0 + j * (kWave * 4) + lane * 4;
      append4(ws, ln, v, e0, kMasks ? mask[j] : group_mask<kTail>(sl, e0), sl);
    }
  }
  // min-p: a new largest value raises the floor.
  if (sl.floor_on && __ballot(ln.amax > ws.top) != 0ull) {
    const uint32_t k = wave_max_u32(ln.amax);
    ws.top = k;
    publish(sl.share + 1, k);
    raise_tau(ws, floor_tau(k, sl.ln_min_p));
  }
  if (ws.cnt >= ws.sel && !ws.spill) select_now(ws, ws.C, ws.C / 4, sl.share);

  if (kSums) {
    const float cm = fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]));
    if (cm > ln.ref) move_ref(ln, cm, sl.scale);
    float g[kU], ga = ln.sa;
#pragma unroll
    for (int j = 0; j < kU; ++j) {
      float e[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float t = (q[j][c] - ln.ref) * sl.scale;
        e[c] = ((mask[j] >> c) & 1u) ? 0.0f : __builtin_amdgcn_exp2f(t);
        ga = fmaf(e[c], -t, ga);
      }
      g[j] = (e[0] + e[1]) + (e[2] + e[3]);
    }
    ln.s = ln.s + (double)((g[0] + g[1]) + (g[2] + g[3]));
    ln.sa = ga;
  }
}

template <bool kVec>
__device__ __forceinline__ void load_chunk(f32x4 (&q)[kU], const float* x, uint32_t c0) {
#pragma unroll
  for (int j = 0; j < kU; ++j) {
    const uint32_t e0 = c0 + j * (kWave * 4) + (threadIdx.x & (kWave - 1)) * 4;
    if (kVec) {
      q[j] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(x + e0));
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) q[j][c] = x[e0 + c];
    }
  }
}
__device__ __forceinline__ void load_tail(f32x4 (&q)[kU], const float* x, uint32_t c0, uint32_t b1) {
#pragma unroll
  for (int j = 0; j < kU; ++j) {
    const uint32_t e0 = c0 + j * (kWave * 4) + (threadIdx.x & (kWave - 1)) * 4;
#pragma unroll
    for (int c = 0; c < 4; ++c) q[j][c] = (e0 + c < b1) ? x[e0 + c] : 0.0f;
  }
}

// The wave's chunks c(i) = c0 + i*kGroupStep, nfull of them full. A load index past the last full
// chunk is clamped to it (or to the zero buffer when there is none), so that every load is issued
// unconditionally and the waits stay exact.
struct Walk {
  uint32_t c0, nfull;
};

// One set of load instructions whatever the case (the base address is selected): two sets writing
// different registers would be merged by copies, which wait for every load in flight.
template <bool kVec>
__device__ __forceinline__ void load_at(f32x4 (&q)[kU], const Slice& sl, const Walk& wk, uint32_t i) {
  const float* base = wk.nfull ? sl.x + (wk.c0 + min(i, wk.nfull - 1) * kGroupStep) : sl.zero;
  load_chunk<kVec>(q, base, 0);
}

// The row's parameter block by scalar loads (a constant-address-space view of device memory): they
// count against their own wait counter, so reading them does not wait for the chunk loads in flight.
__device__ __forceinline__ RowParams load_params(const RowParams* p) {
  struct Words {
    uint32_t w[sizeof(RowParams) / 4];
  } r;
  const __attribute__((address_space(4))) uint32_t* q = (const __attribute__((address_space(4))) uint32_t*)p;
#pragma unroll
  for (uint32_t i = 0; i < sizeof(RowParams) / 4; ++i) r.w[i] = q[i];
  return __builtin_bit_cast(RowParams, r);
}

// Lane i < n_slots reads the row's slot i (others: all ones, so that the wave's minimum is the slots').
__device__ __forceinline__ uint32_t read_slot(const Slice& sl) {
  const uint32_t lane = threadIdx.x & (kWave - 1);
  if (lane < sl.n_slots) return __hip_atomic_load(sl.slots + lane, __ATOMIC_RELAXED, kShareScope);
  return 0xFFFFFFFFu;
}

// The row's shared words as read: the published bound, the slots' minimum (top-k rows: once every
// slot is set, at least k values of the row rank at or above it), and min-p's largest key.
__device__ __forceinline__ void apply_shared(WaveState& ws, const Slice& sl, uint64_t w, uint32_t sv, uint32_t ln_amax) {
  const uint32_t b = __builtin_amdgcn_readfirstlane((uint32_t)w);
  raise_tau(ws, (uint64_t)b << 32);
  if (sl.n_slots) {
    raise_tau(ws, (uint64_t)wave_min_u32(sv) << 32);
    // The wave's slot: the q-th largest of its lanes' largest appended keys (q distinct unmasked
    // values of the wave rank at or above it).
    if (sl.my_slot) {
      const uint32_t t = wave_qth(ln_amax, sl.q);
      if (t) publish(sl.my_slot, t);
    }
  }
  if (sl.floor_on) {
    const uint32_t top = __builtin_amdgcn_readfirstlane((uint32_t)(w >> 32));
    if (top > ws.top) {
      ws.top = top;
      raise_tau(ws, floor_tau(top, sl.ln_min_p));
    }
  }
}

// The walk: qa and qb hold chunks 0 and 1 (as loaded); chunk i+1 is in flight while chunk i is
// worked on, and the row's shared words are read once per kShareEvery chunks; then the partial chunk
// at the slice's end.
template <int kKind, bool kVec>
__device__ __forceinline__ void stream(Lane& ln, WaveState& ws, const Slice& sl, const Walk& wk,
                                       f32x4 (&q)[kDepth][kU]) {
  constexpr bool kShare = kKind != kKindPlain;
  const uint32_t nfull = wk.nfull;
  if (nfull > 0) {
    chunk<kKind, false, true>(ln, ws, sl, q[0], wk.c0);
    // Chunk c sits in buffer c % kDepth; the buffer just worked on takes chunk c - 1 + kDepth before
    // chunk c is worked on, so kDepth - 1 chunks are in flight at every step. The loop runs in steps
    // of kDepth so that every buffer index is a constant.
    for (uint32_t i = 1; i < nfull; i += kDepth) {
#pragma unroll
      for (int j = 0; j < kDepth; ++j) {
        const uint32_t c = i + (uint32_t)j;
        if (c >= nfull) break;
        const bool now = kShare && (c % kShareEvery) == 1;
        const uint64_t w = now ? read_shared(sl.share) : 0ull;
        const uint32_t sv = now ? read_slot(sl) : 0xFFFFFFFFu;
        load_at<kVec>(q[j % kDepth], sl, wk, c - 1 + kDepth);
        chunk<kKind, false, false>(ln, ws, sl, q[(j + 1) % kDepth], wk.c0 + c * kGroupStep);
        if (now) apply_shared(ws, sl, w, sv, ln.amax);
      }
    }
  }
  const uint32_t ct = wk.c0 + nfull * kGroupStep;
  if (ct < sl.b1) {
    f32x4 t[kU];
    load_tail(t, sl.x, ct, sl.b1);
    if (nfull == 0) chunk<kKind, true, true>(ln, ws, sl, t, ct);
    else chunk<kKind, true, false>(ln, ws, sl, t, ct);
  }
}

// One slice (seg) of one row: the body of the scan kernel. tail_list may be null (the rows whose
// slices give up keeping min-p's floor set are then not listed).
template <bool kVec>
// Returns the slice's statistics (in thread 0; as stored).
__device__ __forceinline__ SegStats scan_slice(
    const float* __restrict__ logits, const float* __restrict__ zero, uint64_t row_stride, uint32_t n,
    uint32_t n_seg, uint32_t slice_len, const RowParams* __restrict__ params, RowShare* share,
    const uint32_t* __restrict__ hist_off, const uint32_t* __restrict__ hist_ids,
    const uint32_t* __restrict__ extra_ids, SegStats* __restrict__ stats, uint64_t* __restrict__ cands,
    uint32_t cand_stride, TailList* tail_list, uint32_t row, uint32_t seg) {
  Shared& sh = shm();
  const uint32_t tid = threadIdx.x;
  // The wave's index as a scalar: the walk's bounds and addresses derive from it, and the compiler
  // keeps the stream's loop control in scalar registers only when it knows them uniform.
  const uint32_t lane = tid & (kWave - 1), w = __builtin_amdgcn_readfirstlane(tid / kWave);

  Slice sl;
  sl.x = logits + (uint64_t)row * row_stride;
  sl.zero = zero;
  sl.share = &share[row].bound;
  sl.b0 = seg * slice_len;
  sl.out = cands + ((uint64_t)row * n_seg + seg) * cand_stride;
  sl.room = cand_stride > as_launch::kHistReserve ? cand_stride - as_launch::kHistReserve : 0u;
  sl.b1 = min(sl.b0 + slice_len, n);
  const uint32_t len = sl.b1 - sl.b0;
  Walk wk;
  wk.c0 = sl.b0 + w * kChunk;
  wk.nfull = (wk.c0 + kChunk <= sl.b1) ? (sl.b1 - wk.c0 - kChunk) / kGroupStep + 1 : 0;

  // The set-up, in the order its loads are issued. Every wave's first chunk goes first: at the
  // start of a call the whole GPU's first chunks take a few microseconds to arrive, and everything
  // below happens meanwhile. The parameters and the history's bounds come by scalar loads, which do
  // not wait for the chunk. The history ids follow the first chunk and come back before the second,
  // so that the LDS tables are built while the second is on its way.
  f32x4 q[kDepth][kU];
  load_at<kVec>(q[0], sl, wk, 0u);
  const RowParams p = load_params(params + row);
  uint32_t hb = 0, he = 0;
  if (hist_ids) {
    if (hist_off) {
      hb = hist_off[row];
      he = hist_off[row + 1];
    } else {
      hb = p.hist_begin;
      he = p.hist_begin + p.hist_len;
    }
  }
  const uint32_t extra = extra_ids ? p.extra : 0;
  sl.pen = (p.flags & kFlagPenalties) && (he > hb || extra > 0);
  constexpr int kHistRegs = 8;
  uint32_t hreg[kHistRegs];
#pragma unroll
  for (int k = 0; k < kHistRegs; ++k) {
    const uint32_t h = hb + tid + k * kThreads;
    hreg[k] = (sl.pen && h < he) ? hist_ids[h] : kEmpty;
  }
#pragma unroll
  for (int d = 1; d < kDepth; ++d) load_at<kVec>(q[d], sl, wk, (uint32_t)d);
  if (tid == 0) {
    sh.prm = p;
    sh.hist_out = 0;
    sh.overflow = 0;
    sh.out_n = 0;
    sh.vast = 0;
  }
  // The history tables start empty.
  if (sl.pen) {
    for (uint32_t i = tid; i < (len + 31) / 32; i += kThreads) sh.bitmap[i] = 0;
    for (uint32_t i = tid; i < kHash; i += kThreads) {
      sh.hid[i] = kEmpty;
      sh.hcnt[i] = 0;
    }
  }
  const uint32_t mode = p.mode, flags = p.flags;
  sl.floor_on = mode == kModePartial && p.min_p > 0.0f;
  sl.ln_min_p = p.ln_min_p;
  int kind = kKindPlain;
  if (mode == kModeTopK || mode == kModePartial) {
    kind = (flags & kFlagSumTemp) ? kKindSumTemp : (flags & kFlagSumTop) ? kKindSumTop : kKindCand;
  }
  sl.scale = kind == kKindSumTemp ? (1.0f / p.temp) * kLog2e : kLog2e;
  sl.C = (kind == kKindPlain) ? 0u : max(p.cand, 1u);
  // A top-k row's tau must have k values at or above it; rows without a top-k take the best the
  // first chunk gives.
  sl.first = mode == kModeTopK ? sl.C <= 2u * kWave : true;
  sl.first_rank = mode == kModeTopK ? sl.C : kFirstRankPartial;
  // Top-k rows: the first min(waves of the row, kShareSlots) waves each own a slot.
  sl.slots = share[row].slot;
  sl.n_slots = (mode == kModeTopK && sl.first) ? min(n_seg * kWaves, kShareSlots) : 0u;
  sl.q = sl.n_slots ? (p.top_k + sl.n_slots - 1) / sl.n_slots : 0u;
  sl.my_slot = (seg * kWaves + w < sl.n_slots) ? sl.slots + seg * kWaves + w : nullptr;
  __syncthreads();  // the tables clear, the parameters in LDS

  if (sl.pen) {
    // A history of at most kHistRegs ids per thread is short: its ids go to the table's first
    // kHashPrimary slots (those whose raw values load before the stream) within kPrimaryProbes
    // probes, the rest of the table takes the others. A longer one's ids hash over the whole table:
    // once its distinct ids fill the first part, every id past it would first probe all of it. An
    // id's probe sequence is fixed for the call and slots are never freed, so every thread marking
    // it reaches the same slot.
    const bool long_hist = he - hb > (uint32_t)(kHistRegs * kThreads);
    auto count = [&](uint32_t slot, uint32_t id) {
      const uint32_t prev = atomicCAS(&sh.hid[slot], kEmpty, id);
      if (prev == kEmpty || prev == id) {
        atomicAdd(&sh.hcnt[slot], 1u);
        return true;
      }
      return false;
    };
    auto mark_in = [&](uint32_t id) {  // id in the slice
      const uint32_t off = id - sl.b0;
      atomicOr(&sh.bitmap[off >> 5], 1u << (off & 31u));
      if (long_hist) {
        uint32_t h = (uint32_t)(((uint64_t)(id * 0x85EBCA77u) * kHash) >> 32);
        for (uint32_t probe = 0; probe < kHash; ++probe) {
          if (count(h, id)) return;
          h = (h + 1) & (kHash - 1);
        }
        sh.overflow = 1;
        return;
      }
      uint32_t h = (id * 0x9E3779B1u) >> kPrimaryShift;
      for (uint32_t probe = 0; probe < kPrimaryProbes; ++probe) {
        if (count(h, id)) return;
        h = (h + 1) & (kHashPrimary - 1);
      }
      constexpr uint32_t kRest = kHash - kHashPrimary;
      h = (uint32_t)(((uint64_t)(id * 0x85EBCA77u) * kRest) >> 32);
      for (uint32_t probe = 0; probe < kRest; ++probe) {
        if (count(kHashPrimary + h, id)) return;
        h = h + 1 == kRest ? 0u : h + 1;
      }
      sh.overflow = 1;
    };
    auto mark = [&](uint32_t id) {
      if (id - sl.b0 < len) mark_in(id);
    };
    if (!long_hist) {
#pragma unroll
      for (int k = 0; k < kHistRegs; ++k)
        if (hreg[k] != kEmpty) mark(hreg[k]);
    } else {
      // kHistRegs ids per thread a step, their loads in flight together; each wave packs the ids in
      // the slice (about one in n_seg) into its candidate buffer, which the stream has not begun to
      // use, and marks them with every lane busy.
      uint32_t* pack = reinterpret_cast<uint32_t*>(sh.buf[w]);
      static_assert(kHistRegs * kWave <= 2 * kCapW, "a step's ids fit a wave's buffer");
      for (uint32_t h0 = hb;; h0 += kHistRegs * kThreads) {
        if (h0 != hb) {
#pragma unroll
          for (int k = 0; k < kHistRegs; ++k) {
            const uint32_t h = h0 + tid + k * kThreads;
            hreg[k] = h < he ? hist_ids[h] : kEmpty;
          }
        }
        uint32_t m = 0;
#pragma unroll
        for (int k = 0; k < kHistRegs; ++k) {
          const bool in = hreg[k] - sl.b0 < len;  // kEmpty is past every slice
          const uint64_t bal = __ballot(in);
          if (in) pack[m + lanes_below(bal)] = hreg[k];
          m += (uint32_t)__builtin_popcountll(bal);
        }
        __builtin_amdgcn_wave_barrier();
        for (uint32_t i = lane; i < m; i += kWave) mark_in(pack[i]);
        __builtin_amdgcn_wave_barrier();
        if (h0 + kHistRegs * kThreads >= he) break;
      }
    }
    for (uint32_t h = tid; h < extra; h += kThreads) mark(extra_ids[h]);
  }
  __syncthreads();

  // The raw values of the slice's history ids in each thread's first kHxEarly slots, in flight
  // during the stream; those in its other slots (a long history's) are read after the stream, where
  // their registers cost the stream nothing.
  float hx[kHxEarly];
#pragma unroll
  for (int k = 0; k < kHxEarly; ++k) {
    const uint32_t id = (sl.pen && own_slot(tid, k)) ? sh.hid[tid + k * kThreads] : kEmpty;
    hx[k] = (id != kEmpty) ? sl.x[id] : 0.0f;
  }

  Lane ln;
  ln.nfa = 0.0f;
  ln.gv = 0.0f;
  ln.gi = kNone;
  ln.amax = 0;
  ln.ref = -__builtin_inff();
  ln.s = 0.0;
  ln.sa = 0.0f;
  ln.moves = 0;
  WaveState ws;
  ws.cnt = 0;
  ws.tau = 0;
  ws.tau_f = -__builtin_inff();
  ws.top = 0;
  ws.C = sl.C;
  ws.sel = select_at(sl.C);
  ws.spill = sl.floor_on && sl.C > as_launch::kPartialRank;

  switch (kind) {
    case kKindPlain: stream<kKindPlain, kVec>(ln, ws, sl, wk, q); break;
    case kKindCand: stream<kKindCand, kVec>(ln, ws, sl, wk, q); break;
    case kKindSumTop: stream<kKindSumTop, kVec>(ln, ws, sl, wk, q); break;
    default: stream<kKindSumTemp, kVec>(ln, ws, sl, wk, q); break;
  }

  // The first non-finite index, searched for only when the slice holds one.
  uint32_t nf = kNone;
  if (__syncthreads_or(ln.nfa != ln.nfa)) {
    for (uint32_t e = sl.b0 + tid; e < sl.b1; e += kThreads)
      if (!is_finite_bits(sl.x[e])) {
        nf = e;
        break;
      }
    nf = block_min_u32<kWaves>(nf, sh.red_u);
  }

  // The slice's history values, penalised.
  const bool sums = kind == kKindSumTop || kind == kKindSumTemp;
  uint64_t hpk[kHashPer];
  uint32_t hkey_max = 0, hidv[kHashPer];
#pragma unroll
  for (int k = 0; k < kHashPer; ++k) {
    hpk[k] = 0;
    hidv[k] = (sl.pen && own_slot(tid, k)) ? sh.hid[tid + k * kThreads] : kEmpty;
    if (hidv[k] != kEmpty) {
      const float raw = k < kHxEarly ? hx[k < kHxEarly ? k : 0] : sl.x[hidv[k]];
      const float v = penalize(raw, sh.hcnt[tid + k * kThreads], sh.prm);
      const uint32_t key = total_key(v);
      hpk[k] = pack(key, hidv[k]);
      hkey_max = max(hkey_max, key);
      if (kind == kKindPlain) {
        if (is_finite_bits(v)) greedy_merge(ln.gv, ln.gi, v, hidv[k]);
      } else if (sums) {
        if (v > ln.ref) move_ref(ln, v, sl.scale);
        const float t = (v - ln.ref) * sl.scale;
        const float e = __builtin_amdgcn_exp2f(t);
        ln.s = ln.s + (double)e;
        ln.sa = fmaf(e, -t, ln.sa);
      }
    }
  }

  SegStats st;
  st.nonfinite = nf;
  st.greedy_idx = kNone;
  st.greedy_val = 0.0f;
  st.max_key = 0;
  st.n_cand = 0;
  st.err_rel = 0.0f;
  st.err_abs = 0.0f;
  st.bound = 0;
  st.sum = 0.0;
  st.sum_abs = 0.0;
  st.sum_ref = 0.0f;
  st.vast = 0;

  if (kind == kKindPlain) {
    wave_greedy(ln.gv, ln.gi);
    if (lane == 0) {
      sh.red_f[w] = ln.gv;
      sh.red_u2[w] = ln.gi;
    }
    __syncthreads();
    float gv = sh.red_f[0];
    uint32_t gi = sh.red_u2[0];
    for (int k = 1; k < kWaves; ++k) greedy_merge(gv, gi, sh.red_f[k], sh.red_u2[k]);
    st.greedy_idx = gi;
    st.greedy_val = gv;
    st.max_key = (gi == kNone) ? 0u : total_key(gv);
    st.truncated = sh.overflow ? 2u : 0u;
  } else {
    // One barrier for the slice's bound (the highest wave threshold and the row's shared one), its
    // largest key and its sums' reference.
    const uint64_t* wbuf = sh.buf[w];
    const uint64_t shared = read_shared(sl.share);
    const uint32_t shared_b = __builtin_amdgcn_readfirstlane((uint32_t)shared);
    const uint32_t shared_top = __builtin_amdgcn_readfirstlane((uint32_t)(shared >> 32));
    const uint32_t kmax = wave_max_u32(max(hkey_max, ln.amax));
    const uint32_t rk = wave_max_u32(ln.ref > -__builtin_inff() ? total_key(ln.ref) : 0u);
    if (lane == 0) {
      sh.red_p[w] = max(ws.tau, (uint64_t)shared_b << 32);
      sh.red_u2[w] = kmax;
      sh.red_u[w] = rk;
    }
    __syncthreads();
    uint64_t bound = sh.red_p[0];
    uint32_t mk = sh.red_u2[0], rkey = sh.red_u[0];
    for (int k = 1; k < kWaves; ++k) {
      bound = max(bound, sh.red_p[k]);
      mk = max(mk, sh.red_u2[k]);
      rkey = max(rkey, sh.red_u[k]);
    }
    st.max_key = mk;
    st.vast = sh.vast;
    // A min-p row's slice whose bound lies above its floor (from the largest value it knows the row
    // to hold) did not keep every value above the floor: the row is flagged for S's sums.
    // The first slice to flag the row lists it.
    if (sl.floor_on && tid == 0 && bound > floor_tau(max(mk, shared_top), sl.ln_min_p)) {
      const uint32_t was = __hip_atomic_fetch_max(&reinterpret_cast<RowShare*>(sl.share)->gave_up, 1u,
                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (was == 0u && tail_list) {
        const uint32_t i = __hip_atomic_fetch_add(&tail_list->count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (i < kTailListMax) {
          tail_list->rows[i] = row;
          tail_list->help[i] = sh.prm.help;
        }
      }
    }

    // Candidates: those spilled during the stream (left where they are: some may rank below the bound,
    // and the finish kernel drops every candidate below the row's bound as it loads them), every
    // buffered value >= bound, wave by wave, then the history values >= bound. When they would not fit
    // the slice's slots, each wave first keeps only its share.
    const uint32_t spilled = sh.out_n;
    uint32_t all = 0, hall = 0;
    for (int pass = 0; pass < 2; ++pass) {
      uint32_t mine = 0;
      for (uint32_t i = lane; i < ws.cnt; i += kWave) mine += wbuf[i] >= bound ? 1u : 0u;
      mine = wave_sum_u32(mine);
      uint32_t hmine = 0;
#pragma unroll
      for (int k = 0; k < kHashPer; ++k) hmine += (hpk[k] != 0ull && hpk[k] >= bound) ? 1u : 0u;
      hmine = wave_sum_u32(hmine);
      __syncthreads();
      if (lane == 0) {
        sh.red_u3[w] = mine;
        sh.red_u[w] = hmine;
      }
      __syncthreads();
      all = 0;
      hall = 0;
      for (int k = 0; k < kWaves; ++k) {
        all += sh.red_u3[k];
        hall += sh.red_u[k];
      }
      if (pass == 1 || spilled + all + hall <= cand_stride) break;
      const uint32_t used = spilled + hall;
      const uint32_t share = cand_stride > used + 4u * kWaves ? (cand_stride - used) / kWaves : 1u;
      if (ws.cnt > share) select_now(ws, share, 0u, nullptr);
      __syncthreads();
      if (lane == 0) sh.red_p[w] = ws.tau;
      __syncthreads();
      for (int k = 0; k < kWaves; ++k) bound = max(bound, sh.red_p[k]);
    }
    uint32_t run = spilled;
    for (int k = 0; k < (int)w; ++k) run += sh.red_u3[k];
    uint64_t* out = sl.out;
    for (uint32_t i0 = 0; i0 < ws.cnt; i0 += kWave) {
      const uint32_t i = i0 + lane;
      const bool take = i < ws.cnt && wbuf[i] >= bound;
      const uint64_t m = __ballot(take);
      const uint32_t pos = run + lanes_below(m);
      if (take && pos < cand_stride) out[pos] = wbuf[i];
      run += (uint32_t)__popcll(m);
    }
#pragma unroll
    for (int k = 0; k < kHashPer; ++k) {
      if (hpk[k] != 0ull && hpk[k] >= bound) {
        const uint32_t pos = spilled + all + atomicAdd(&sh.hist_out, 1u);
        if (pos < cand_stride) out[pos] = hpk[k];
      }
    }
    st.bound = bound;
    st.n_cand = min(spilled + all + hall, cand_stride);
    st.truncated = ((sh.overflow || spilled + all + hall > cand_stride) ? 2u : 0u) | (bound != 0 ? 1u : 0u);

    if (sums) {
      // Each lane's sums moved from its reference to the slice's largest one, m.
      const float m = rkey ? key_value(rkey) : 0.0f;
      double s = 0.0, sa = 0.0;
      if (ln.s != 0.0) {
        const float dt = (ln.ref - m) * sl.scale;
        const float sc = __builtin_amdgcn_exp2f(dt);
        s = ln.s * (double)sc;
        sa = (double)(sc * fmaf((float)ln.s, fabsf(dt), ln.sa));
      }
      s = wave_sum_f64(s);
      sa = wave_sum_f64(sa);
      const uint32_t moves = wave_max_u32(ln.moves);
      if (lane == 0) {
        sh.red_d[w] = s;
        sh.red_d2[w] = sa;
        sh.red_u2[w] = moves;
      }
      __syncthreads();
      double ts = sh.red_d[0], tsa = sh.red_d2[0];
      uint32_t tm = sh.red_u2[0];
      for (int k = 1; k < kWaves; ++k) {
        ts = __dadd_rn(ts, sh.red_d[k]);
        tsa = __dadd_rn(tsa, sh.red_d2[k]);
        tm = max(tm, sh.red_u2[k]);
      }
      st.sum = ts;
      st.sum_ref = m;
      // sum_abs in units of d = t * ln(2); it was kept in f32 (a lane folds a few hundred terms): a
      // 2^-10 margin covers its roundings.
      st.sum_abs = tsa * 0.69314718055994531 * (1.0 + 0x1p-10);
      // Per term: the exp's own error once for the term, once per move of its lane's reference and
      // once for the move to m; the chunk's f32 tree (4 levels); the f64 folds (the lane's chunks
      // one by one, then 10 levels of wave and block adds) are far below that.
      st.err_rel = kExpUlp * 0x1p-23f * (float)(tm + 2) + 4.0f * 0x1p-24f +
                   0x1p-53f * (float)((len + kChunk - 1) / kChunk + 16);
      st.err_abs = 5.0f * 0x1p-24f * 1.01f;
    }
  }
  if (tid == 0) stats[(uint64_t)row * n_seg + seg] = st;
  return st;
}

}  // namespace AS_SCAN_NS
}  // namespace
