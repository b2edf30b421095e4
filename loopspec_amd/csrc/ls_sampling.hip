// (a) logit processing and (c) lossless speculative sampling for gfx950.
//
// One persistent launch does the whole path (plus a penalty-bitmap pre-pass
// when a repetition penalty is on, and a dense-output pass in filter mode).
// Workgroups of 256 lanes stream (row, chunk) items of kChunk logits in
// row-major order, with the next item's loads in flight while the current one
// is processed. Per item:
//   chunk max m_j of the penalised logits, mc_j = RN(m_j c) (c = log2 e / T),
//   e = exp2q(fma(x, c, -mc_j)), the chunk mass M_j (binary32, fixed
//   summation order), a histogram of the binary exponents of e, and the
//   chunk's largest entries (every e >= 2^(1-K_j), at most cap of them, K_j
//   the most leading exponent bins that fit) compacted in index order into
//   the workspace; then
//   each wave arrives on the row's counter.
// The wave that arrives last makes its workgroup finalise the row: row max,
// f_j = exp2q(mc_j - max), S = sum f_j M_j, g_j = RN(f_j / S), p = RN(e g_j)
// for the candidates, and the exact top-p cutoff by a radix select on the
// binary32 bits of p with 2^-46 fixed-point masses (replacing sort + cumsum +
// searchsorted, distributions.py:59-70). The cutoff is valid for the whole
// row iff it exceeds every p outside the candidates; otherwise the row is
// re-streamed for an exact select. Then, per mode:
//   spec    publish the row's statistics and the filtered probability of its
//           draft token, arrive on the batch element's counter; the last of
//           its 2k+1 rows runs the chain verify: accept tests, then the
//           residual or bonus draw over the target row's candidates;
//   sample  draw one token from the filtered distribution;
//   dense   publish the statistics for dense_kernel, which writes p and/or the
//           filtered, renormalised rows.
// The arithmetic is the declared arithmetic of ls_numerics.hpp (restated by
// oracle/sampling.py), so every output is bit-identical to the oracle's.
#include "ls_common.hpp"
#include "ls_numerics.hpp"
#include "ls_runtime.hpp"

namespace ls {
namespace {

constexpr int kChunk = 2048;                 // softmax chunk (declared arithmetic)
constexpr int kChunkShift = 11;
constexpr int kCB = 256;                     // row kernel lanes
constexpr int kCW = kCB / kWave;
constexpr int kPerLane = kChunk / kWave;     // 32 elements per lane: one wave per chunk
constexpr int kChunkCand = 64;               // candidate slots per chunk in the workspace
constexpr int kOctBins = 16;                 // exponent bins of e
constexpr int kHistStride = kOctBins + 1;    // lane-private bins, padded against bank conflicts
constexpr int kRowCand = 2048;               // candidate slots of a row
constexpr int kSlotsPerLane = kRowCand / kCB;
constexpr int kMaxChunks = 128;              // vocab <= 262144
constexpr int kMaxVocab = kMaxChunks * kChunk;
constexpr int kBins = 2048;                  // radix digits per round
constexpr int kBinsPerLane = kBins / kCB;
constexpr int kGather = kWave;               // bucket size finished by one wave
constexpr int kCounterStride = 16;           // arrival counters one 64-byte line apart
constexpr int kChunkWavesPerCu = 12;         // resident chunk waves per CU (LDS-bound)
constexpr int64_t kMaxRows = 65536;
constexpr int64_t kMaxSpecBatch = 16384;
constexpr uint32_t kNone = 0xffffffffu;

enum Mode : int { kModeSpec = 0, kModeSample = 1, kModeDense = 2 };
enum RowFlag : uint32_t { kFlagUnfiltered = 1u, kFlagDense = 2u, kFlagSlow = 4u };
enum ChunkFlag : uint32_t { kChunkComplete = 1u, kChunkHasTok = 2u };

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Per-chunk result, published by the chunk's workgroup.
struct ChunkRec {
  float mc;         // RN(chunk max * c)
  int32_t K;        // candidates are the e >= 2^(1-K) (every e > 0 when complete)
  uint32_t n;       // candidates written
  uint32_t flags;
  float mass;       // chunk mass M_j
  float e_tok;      // e of the row's draft token when it lies in this chunk
  uint32_t pad0, pad1;
};
static_assert(sizeof(ChunkRec) == 32, "ChunkRec layout");

// Published per-row statistics.
struct RowStat {
  float mcmax;      // row max of mc_j
  float s;          // normaliser S
  float cutoff;     // top-p cutoff value (0 when unfiltered)
  float mass;       // binary32 retained mass (renormaliser; 1 when unfiltered)
  uint32_t flags;
  float p_tok;      // filtered probability of the row's draft token
  uint64_t mass_fx; // exact retained mass
};
static_assert(sizeof(RowStat) == 32, "RowStat layout");

struct SampParams {
  const char* base0;           // target / row logits
  int64_t bstride0, pstride0;  // bytes
  const char* base1;           // draft logits (spec mode)
  int64_t bstride1, pstride1;
  int rpg;                     // rows per group: spec 2k+1, else 1
  int k;                       // spec: draft positions; 0 otherwise
  int vocab;
  int nch;                     // chunks per row
  int cap, cap_log2;           // candidates kept per chunk (a power of two)
  int bm_words;                // penalty bitmap words per group
  int items;                   // rows * nch
  float c;                     // exponent scale RN(log2e * RN(1/T))
  float pen, inv_pen;
  int use_pen;
  float top_p;                 // >= 1: unfiltered
  const float* top_p_rows;     // optional per-row top_p (dense mode)
  const int32_t* hist;
  int64_t hist_stride;
  const int32_t* hist_len;
  // spec mode
  const int64_t* draft_tokens;  // [B, k]
  const float* uniforms;        // [B, 2k+1]
  int32_t* accept_len;
  int64_t* tokens;              // [B, k+1]
  // sample mode
  const float* row_uniforms;    // [rows]
  int64_t* row_tokens;          // [rows]
  // dense mode
  float* probs_out;
  int64_t probs_stride;         // elements
  float* filt_out;
  int64_t filt_stride;
  float* cutoff_out;
  float* mass_out;
  // workspace
  ChunkRec* chunks;             // [rows, nch]
  uint64_t* cands;              // [rows, nch, kChunkCand] of (idx << 32 | bits(e))
  RowStat* stats;               // [rows]
  uint32_t* row_cnt;            // [kMaxRows * kCounterStride]
  uint32_t* grp_cnt;            // [kMaxSpecBatch * kCounterStride]
  uint32_t* bitmap;             // [groups, bm_words] penalty bits
  int64_t* draws;               // spec: [B, k+1] residual draws, then the bonus draw
};

// Row jr of group g: spec rows are target positions 0..k, then draft 0..k-1.
__device__ __forceinline__ const char* row_of(const SampParams& p, int64_t g, int jr) {
  if (jr <= p.k) return p.base0 + g * p.bstride0 + jr * p.pstride0;
  return p.base1 + g * p.bstride1 + (jr - p.k - 1) * p.pstride1;
}

// The draft token whose probability row jr of group g contributes to the
// accept test (target position i and draft position i both test x_i); -1 for
// the bonus row and outside spec mode.
__device__ __forceinline__ int64_t row_token(const SampParams& p, int64_t g, int jr) {
  if (p.k == 0 || jr == p.k) return -1;
  const int i = jr < p.k ? jr : jr - p.k - 1;
  return p.draft_tokens[g * p.k + i];
}

__device__ __forceinline__ bool bit_of(const uint32_t* bm, int idx) { return (bm[idx >> 5] >> (idx & 31)) & 1u; }

// ---------------------------------------------------------------------------
// Wave sums in the declared pairwise order (lanes 2i and 2i+1 first, then
// pairs of those ...): quad_perm swaps for distance 1 and 2, then the half-row
// and row mirrors (equivalent to distance 4 and 8 once every quad / half-row
// holds one value), then the row broadcasts.
// ---------------------------------------------------------------------------
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_add(float v) {
  return __uint_as_float(dpp32<CTRL, ROWS>(0u, __float_as_uint(v))) + v;
}

// Pairwise sum over the 16 lanes of each row (every lane of the row gets it).
__device__ __forceinline__ float row_tree_sum(float v) {
  v = dpp_add<kDppQuadXor1, 0xf>(v);
  v = dpp_add<kDppQuadXor2, 0xf>(v);
  v = dpp_add<kDppRowHalfMirror, 0xf>(v);
  v = dpp_add<kDppRowMirror, 0xf>(v);
  return v;
}

// Pairwise sum over the 64 lanes (wave-uniform result).
__device__ __forceinline__ float wave_tree_sum(float v) {
  v = row_tree_sum(v);
  v = dpp_add<kDppRowBcast15, 0xa>(v);  // rows 1, 3: r0 + r1, r2 + r3
  v = dpp_add<kDppRowBcast31, 0xc>(v);  // row 3: (r0 + r1) + (r2 + r3)
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_uint(v), kWave - 1));
}

// Pairwise sum over lanes 0..31 (wave-uniform result).
__device__ __forceinline__ float half_tree_sum(float v) {
  v = row_tree_sum(v);
  v = dpp_add<kDppRowBcast15, 0xa>(v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_uint(v), 31));
}

// Pairwise sum of N values held by one lane, adjacent pairs first.
template <int N>
__device__ __forceinline__ float lane_tree_sum(float (&a)[N]) {
#pragma unroll
  for (int w = 1; w < N; w *= 2) {
#pragma unroll
    for (int i = 0; i < N; i += 2 * w) a[i] = a[i] + a[i + w];
  }
  return a[0];
}

// ---------------------------------------------------------------------------
// Shared memory: the chunk phase and the row / tail phases share one region.
// ---------------------------------------------------------------------------
struct ChunkSh {
  float est[kChunk];                   // e of the chunk, 16-byte slots XOR-swizzled
  uint32_t hist[kWave * kHistStride];  // lane-private exponent bins
};

struct FinSh {
  uint64_t slot[kRowCand];             // the row's candidate slots (idx << 32 | bits)
  union {
    uint64_t H[kBins];                 // radix bins
    uint64_t slot_d[kRowCand];         // tail: the draft row's candidate slots
    float w[kRowCand];                 // tail: draw weights per slot
    uint64_t words64[kBins];           // tail: row statistics (4 words each)
  };
  float g[2][kMaxChunks];
  float mcj[2][kMaxChunks];
  uint32_t n[2][kMaxChunks];
  uint32_t gbits[kGather];
  uint64_t gw[kGather];
  uint32_t gcount;
  uint64_t statw[8];                   // residual: both rows' statistics
  float tokp[2 * 64 + 1];              // accept chain: P / Q of the draft tokens
  int64_t tokd[64 + 1];                // accept chain: the published draws
};

struct Shared {
  FinSh f;
  uint64_t red[kCW];
  uint64_t u64s[8];
  uint32_t u32s[8];
  float f32s[8];
};

// Physical float index of element v of the chunk in the e-store.
__device__ __forceinline__ int est_index(int v) {
  const int s = v >> 2;
  return ((s ^ ((s >> 3) & 7)) << 2) | (v & 3);
}

// Exclusive scan in lane order over the workgroup; *total receives the sum.
__device__ __forceinline__ uint64_t block_excl_scan(uint64_t v, uint64_t* smem, uint64_t* total) {
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  const uint64_t inc = wave_scan_add_u64(v);
  __syncthreads();
  if (lane == kWave - 1) smem[wid] = inc;
  __syncthreads();
  uint64_t base = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kCW; ++i) {
    const uint64_t s = smem[i];
    base += i < wid ? s : 0;
    tot += s;
  }
  *total = tot;
  return base + inc - v;
}

__device__ __forceinline__ uint64_t block_sum(uint64_t v, uint64_t* smem) {
  uint64_t tot;
  (void)block_excl_scan(v, smem, &tot);
  return tot;
}

__device__ __forceinline__ uint64_t pack2(uint32_t lo, uint32_t hi) {
  return static_cast<uint64_t>(lo) | (static_cast<uint64_t>(hi) << 32);
}
__device__ __forceinline__ uint64_t pack2f(float lo, float hi) { return pack2(__float_as_uint(lo), __float_as_uint(hi)); }
__device__ __forceinline__ float lo_f(uint64_t v) { return __uint_as_float(static_cast<uint32_t>(v)); }
__device__ __forceinline__ float hi_f(uint64_t v) { return __uint_as_float(static_cast<uint32_t>(v >> 32)); }

__device__ __forceinline__ void put_rec(ChunkRec* dst, const ChunkRec& v) {
  uint64_t* d = reinterpret_cast<uint64_t*>(dst);
  store_sc64(d + 0, pack2(__float_as_uint(v.mc), static_cast<uint32_t>(v.K)));
  store_sc64(d + 1, pack2(v.n, v.flags));
  store_sc64(d + 2, pack2f(v.mass, v.e_tok));
}
__device__ __forceinline__ ChunkRec get_rec(const ChunkRec* src) {
  const uint64_t* s = reinterpret_cast<const uint64_t*>(src);
  const uint64_t a = load_sc64(s + 0), b = load_sc64(s + 1), c = load_sc64(s + 2);
  ChunkRec v;
  v.mc = lo_f(a);
  v.K = static_cast<int32_t>(a >> 32);
  v.n = static_cast<uint32_t>(b);
  v.flags = static_cast<uint32_t>(b >> 32);
  v.mass = lo_f(c);
  v.e_tok = hi_f(c);
  v.pad0 = v.pad1 = 0;
  return v;
}
__device__ __forceinline__ void put_stat(RowStat* dst, const RowStat& v) {
  uint64_t* d = reinterpret_cast<uint64_t*>(dst);
  store_sc64(d + 0, pack2f(v.mcmax, v.s));
  store_sc64(d + 1, pack2f(v.cutoff, v.mass));
  store_sc64(d + 2, pack2(v.flags, __float_as_uint(v.p_tok)));
  store_sc64(d + 3, v.mass_fx);
}
// The four 64-bit words of a published RowStat and the struct they encode.
__device__ __forceinline__ RowStat stat_of(uint64_t a, uint64_t b, uint64_t c, uint64_t d) {
  RowStat v;
  v.mcmax = lo_f(a);
  v.s = hi_f(a);
  v.cutoff = lo_f(b);
  v.mass = hi_f(b);
  v.flags = static_cast<uint32_t>(c);
  v.p_tok = hi_f(c);
  v.mass_fx = d;
  return v;
}

// ===========================================================================
// bitmap_kernel: the penalty bitmap of each group's token history
// ===========================================================================
constexpr int kBmB = 1024;

__global__ __launch_bounds__(kBmB) void bitmap_kernel(const SampParams p) {
  __shared__ uint32_t bm[kMaxVocab / 32];
  const int t = threadIdx.x;
  const int64_t g = blockIdx.x;
  const int words = p.bm_words;
  for (int w = t; w < words; w += kBmB) bm[w] = 0u;
  __syncthreads();
  const int n = p.hist_len[g];
  const int32_t* h = p.hist + g * p.hist_stride;
  for (int i = t; i < n; i += kBmB) {
    const int id = h[i];
    if (static_cast<unsigned>(id) < static_cast<unsigned>(p.vocab))
      __hip_atomic_fetch_or(&bm[id >> 5], 1u << (id & 31), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  __syncthreads();
  uint32_t* out = p.bitmap + g * words;
  for (int w = t; w < words; w += kBmB) out[w] = bm[w];
}

// ===========================================================================
// Chunk phase
// ===========================================================================

// Loads of one chunk (lanes past the chunk end re-read its last vector), plus,
// with a penalty, the bitmap word of each vector (the bits of a 16-byte vector
// always sit in one 32-bit word).
template <int DT, int NVC>
__device__ __forceinline__ void load_chunk(const SampParams& p, int item, u32x4 (&d)[NVC], uint32_t (&pw)[NVC]) {
  constexpr int EPV = Elem<DT>::kPerVec;
  const int r = item / p.nch;
  const int cj = item - r * p.nch;
  const int g = r / p.rpg;
  const int jr = r - g * p.rpg;
  const int c0 = cj * kChunk;
  const int nel = p.vocab - c0 < kChunk ? p.vocab - c0 : kChunk;
  const int nvc = nel / EPV;
  const u32x4* src = reinterpret_cast<const u32x4*>(row_of(p, g, jr)) + c0 / EPV;
#pragma unroll
  for (int u = 0; u < NVC; ++u) {
    const int v = u * kWave + static_cast<int>(threadIdx.x);
    d[u] = __builtin_nontemporal_load(src + (v < nvc ? v : nvc - 1));
  }
  if (p.use_pen) {
    const uint32_t* bm = p.bitmap + static_cast<int64_t>(g) * p.bm_words + c0 / 32;
#pragma unroll
    for (int u = 0; u < NVC; ++u) pw[u] = bm[((u * kWave + static_cast<int>(threadIdx.x)) * EPV) >> 5];
  }
}

__device__ __forceinline__ int64_t item_token(const SampParams& p, int item) {
  if (p.k == 0) return -1;
  const int r = item / p.nch;
  const int g = r / p.rpg;
  return row_token(p, g, r - g * p.rpg);
}

// One chunk, processed by one wave: no workgroup barriers (the wave's LDS
// accesses are ordered; s_barrier of a one-wave workgroup only fences).
template <int DT, int NVC>
__device__ __forceinline__ void process_chunk(const SampParams& p, ChunkSh& cs, int item, const u32x4 (&d)[NVC],
                                              const uint32_t (&pw)[NVC], int64_t tok) {
  constexpr int EPV = Elem<DT>::kPerVec;
  constexpr int NE = NVC * EPV;
  static_assert(NE == kPerLane, "32 elements per lane");
  // lane-derived values are recomputed per item (not hoisted out of the
  // persistent loop)
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  const int r = item / p.nch;
  const int cj = item - r * p.nch;
  const int c0 = cj * kChunk;
  const int nel = p.vocab - c0 < kChunk ? p.vocab - c0 : kChunk;
  const int nvc = nel / EPV;
  const bool full = nvc == NVC * kWave;  // only a row's last chunk can be partial

  // 1. penalised logits (-inf past the row end) and the chunk max
  float x[NE];
#pragma unroll
  for (int u = 0; u < NVC; ++u) {
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      float l = vec_elem<DT>(d[u], e);
      if (p.use_pen && ((pw[u] >> ((((u * kWave + t) * EPV) & 31) + e)) & 1u)) l = l < 0.0f ? l * p.pen : l * p.inv_pen;
      x[u * EPV + e] = l;
    }
  }
  if (!full) {
#pragma unroll
    for (int u = 0; u < NVC; ++u) {
      if (u * kWave + t >= nvc) {
#pragma unroll
        for (int e = 0; e < EPV; ++e) x[u * EPV + e] = -__builtin_inff();
      }
    }
  }
  float mx = x[0];
#pragma unroll
  for (int i = 1; i < NE; ++i) mx = nmax(mx, x[i]);
  const float m = wave_max_f32(mx);
  const float mc = m * p.c;
  const float nmc = -mc;

  // 2. e in place, lane-private exponent bins, e-store. Bin b holds e in
  // [2^-b, 2^(1-b)) (bin 0: e >= 1; the last bin: everything smaller); lanes
  // past the row end are not counted.
  const int hbase = t * kHistStride + 127;
#pragma unroll
  for (int u = 0; u < NVC; ++u) {
    const bool in = full || u * kWave + t < nvc;
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      const float ev = exp2q(__builtin_fmaf(x[u * EPV + e], p.c, nmc));
      x[u * EPV + e] = ev;
      const int be = static_cast<int>(__float_as_uint(ev) >> 23);
      const int bc = __builtin_elementwise_min(__builtin_elementwise_max(be, 127 - (kOctBins - 1)), 127);
      if (in) __hip_atomic_fetch_add(&cs.hist[hbase - bc], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
#pragma unroll
    for (int h = 0; h < EPV / 4; ++h) {
      const int s = (u * kWave + t) * (EPV / 4) + h;
      const int ps = s ^ ((s >> 3) & 7);
      f32x4 v;
      v.x = x[u * EPV + 4 * h + 0];
      v.y = x[u * EPV + 4 * h + 1];
      v.z = x[u * EPV + 4 * h + 2];
      v.w = x[u * EPV + 4 * h + 3];
      *reinterpret_cast<f32x4*>(&cs.est[ps * 4]) = v;
    }
  }
  // chunk mass: each lane's 32 e pairwise, then the lanes pairwise
  const float mass = wave_tree_sum(lane_tree_sum(x));
  __syncthreads();

  // 3. bin totals: lane (b, q) sums bin b of lanes 16q..16q+15 and clears it
  uint32_t bc;
  {
    const int b = t & (kOctBins - 1), q = t >> 4;
    uint32_t sb = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      sb += __hip_atomic_exchange(&cs.hist[(16 * q + i) * kHistStride + b], 0u, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_WORKGROUP);
    sb += __shfl_xor(sb, 16);
    sb += __shfl_xor(sb, 32);
    bc = t < kOctBins ? sb : 0u;
  }
  // lane-contiguous e: elements [32t, 32t + 32) (index order within the lane)
  float ec[kPerLane];
#pragma unroll
  for (int q = 0; q < kPerLane / 4; ++q) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(&cs.est[(8 * t + (q ^ (t & 7))) * 4]);
    ec[4 * q + 0] = v.x;
    ec[4 * q + 1] = v.y;
    ec[4 * q + 2] = v.z;
    ec[4 * q + 3] = v.w;
  }
  const bool has_tok = tok >= c0 && tok < c0 + nel;
  float e_tok = 0.0f;
  if (has_tok) e_tok = cs.est[est_index(static_cast<int>(tok - c0))];

  // 4. K: the number of leading exponent bins holding at most cap entries
  const uint32_t binc = wave_scan_add_u32(bc);
  const int K = __builtin_popcountll(__ballot(t < kOctBins && binc <= static_cast<uint32_t>(p.cap)));
  const float th = K >= kOctBins ? __uint_as_float(1u) : (K == 0 ? __builtin_inff() : __builtin_ldexpf(1.0f, 1 - K));
  // 5. candidate mask (bit 31 - i <-> element 32t + i), offsets
  uint32_t mask = 0;
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) mask = (mask << 1) | (ec[i] >= th ? 1u : 0u);
  const uint32_t cnt = static_cast<uint32_t>(__builtin_popcount(mask));
  const uint32_t incl = wave_scan_add_u32(cnt);
  const uint32_t total = lane_bcast_u32(incl, kWave - 1);
  uint32_t pos = incl - cnt;
  // 6. candidates, in index order
  uint64_t* out = p.cands + (static_cast<int64_t>(r) * p.nch + cj) * kChunkCand;
  const uint32_t ibase = static_cast<uint32_t>(c0 + kPerLane * t);
  while (mask) {
    const int i = __builtin_clz(mask);
    const uint32_t eb = __float_as_uint(cs.est[(8 * t + ((i >> 2) ^ (t & 7))) * 4 + (i & 3)]);
    out[pos] = (static_cast<uint64_t>(ibase + static_cast<uint32_t>(i)) << 32) | eb;
    ++pos;
    mask &= 0x7fffffffu >> i;
  }
  if (t == 0) {
    ChunkRec rec;
    rec.mc = mc;
    rec.K = K;
    rec.n = total;
    rec.flags = (K >= kOctBins ? kChunkComplete : 0u) | (has_tok ? kChunkHasTok : 0u);
    rec.mass = mass;
    rec.e_tok = e_tok;
    rec.pad0 = rec.pad1 = 0;
    p.chunks[static_cast<int64_t>(r) * p.nch + cj] = rec;
  }
  __syncthreads();  // the e-store and bins are rewritten by the next item
}

// Persistent over (row, chunk) items in row-major order, double-buffered: the
// next item's loads are in flight while the current one is processed.
template <int DT>
__global__ __launch_bounds__(kWave, kChunkWavesPerCu) void chunk_kernel(const SampParams p) {
  constexpr int EPV = Elem<DT>::kPerVec;
  constexpr int NVC = kChunk / (kWave * EPV);  // vectors per lane: 8 (f32) or 4
  __shared__ ChunkSh cs;
  const int t = threadIdx.x;
  for (int i = t; i < kWave * kHistStride; i += kWave) cs.hist[i] = 0u;
  __syncthreads();
  int item = blockIdx.x;
  if (item >= p.items) return;
  u32x4 cur[NVC], nxt[NVC];
  uint32_t pcur[NVC] = {}, pnxt[NVC] = {};
  load_chunk<DT, NVC>(p, item, cur, pcur);
  int64_t tcur = item_token(p, item), tnxt = -1;
  while (true) {
    const int next = item + static_cast<int>(gridDim.x);
    if (next < p.items) {
      load_chunk<DT, NVC>(p, next, nxt, pnxt);
      tnxt = item_token(p, next);
    }
    process_chunk<DT, NVC>(p, cs, item, cur, pcur, tcur);
    if (next >= p.items) break;
    // register moves (the empty asm keeps the copy from becoming a memcpy of
    // the arrays, which would put them in scratch)
#pragma unroll
    for (int u = 0; u < NVC; ++u) {
      u32x4 v = nxt[u];
      asm volatile("" : "+v"(v));
      cur[u] = v;
      pcur[u] = pnxt[u];
    }
    tcur = tnxt;
    item = next;
  }
}

// ===========================================================================
// Row phase
// ===========================================================================

// Wave 0: from the chunk records of a row (lane l holds records 2l and
// 2l+1) compute the row max, S and g_j (kept in fs.g / fs.mcj / fs.n [slot]),
// the bound on every p outside the candidates, and p of the draft token.
struct RowScale {
  float mcmax, s, p_bound, p_tok;
  bool has_tok;
};

__device__ __forceinline__ float chunk_bound(const ChunkRec& rec, float gj) {
  if (rec.flags & kChunkComplete) return 0.0f;
  return rec.K > 0 ? __builtin_ldexpf(1.0f, 1 - rec.K) * gj : __builtin_inff();
}

__device__ __forceinline__ RowScale row_scale(FinSh& fs, int slot, const ChunkRec& ra, const ChunkRec& rb, int nch) {
  const int lane = threadIdx.x & (kWave - 1);
  const int ja = 2 * lane, jb = ja + 1;
  const bool ia = ja < nch, ib = jb < nch;
  RowScale rs;
  rs.mcmax = wave_max_f32(nmax(ia ? ra.mc : -__builtin_inff(), ib ? rb.mc : -__builtin_inff()));
  const float fa = ia ? exp2q(ra.mc - rs.mcmax) : 0.0f;
  const float fb = ib ? exp2q(rb.mc - rs.mcmax) : 0.0f;
  // slots 2l and 2l+1 are the first pairwise level of the normaliser's sum
  rs.s = wave_tree_sum((ia ? fa * ra.mass : 0.0f) + (ib ? fb * rb.mass : 0.0f));
  const float ga = fa / rs.s, gb = fb / rs.s;
  if (ia) {
    fs.g[slot][ja] = ga;
    fs.mcj[slot][ja] = ra.mc;
    fs.n[slot][ja] = ra.n;
  }
  if (ib) {
    fs.g[slot][jb] = gb;
    fs.mcj[slot][jb] = rb.mc;
    fs.n[slot][jb] = rb.n;
  }
  rs.p_bound = wave_max_f32(__builtin_fmaxf(ia ? chunk_bound(ra, ga) : 0.0f, ib ? chunk_bound(rb, gb) : 0.0f));
  const bool ta = ia && (ra.flags & kChunkHasTok), tb = ib && (rb.flags & kChunkHasTok);
  rs.has_tok = __ballot(ta || tb) != 0;
  rs.p_tok = wave_max_f32(ta ? ra.e_tok * ga : (tb ? rb.e_tok * gb : -1.0f));
  return rs;
}

// g_j from published row statistics (mcmax, S), two chunks per lane.
__device__ __forceinline__ void row_g(FinSh& fs, int slot, const ChunkRec& ra, const ChunkRec& rb, int nch,
                                      float mcmax, float s) {
  const int lane = threadIdx.x & (kWave - 1);
  const int ja = 2 * lane, jb = ja + 1;
  if (ja < nch) {
    fs.g[slot][ja] = exp2q(ra.mc - mcmax) / s;
    fs.mcj[slot][ja] = ra.mc;
    fs.n[slot][ja] = ra.n;
  }
  if (jb < nch) {
    fs.g[slot][jb] = exp2q(rb.mc - mcmax) / s;
    fs.mcj[slot][jb] = rb.mc;
    fs.n[slot][jb] = rb.n;
  }
}

// Chunk records 2l and 2l+1 of row r for lane l of wave 0.
__device__ __forceinline__ void load_recs(const SampParams& p, int64_t r, ChunkRec* ra, ChunkRec* rb) {
  const int lane = threadIdx.x & (kWave - 1);
  const int ja = 2 * lane, jb = ja + 1;
  if (ja < p.nch) *ra = p.chunks[r * p.nch + ja];
  if (jb < p.nch) *rb = p.chunks[r * p.nch + jb];
}

__device__ __forceinline__ uint32_t digit_of(uint32_t bits, int shift, uint32_t dmask) {
  const uint32_t d = (bits >> shift) & dmask;
  return d < kBins ? d : kBins - 1;
}

// Exact top-p cutoff over a set whose elements visit(f) passes to f(bits, w)
// (bits of p > 0, w = fx46(p)): c = max{v : sum_{p >= v} w >= thr}, and the
// mass kept. Up to three radix rounds on the bits of p (12, 11 and 8 bits
// from the top; fs.H must be zero on entry); after each round a bucket of at
// most kGather entries is finished by one wave. Returns false if the set's
// total mass is below thr.
template <typename Visit>
__device__ bool radix_select(Shared& sh, uint64_t thr, Visit visit, float* cutoff, uint64_t* mass) {
  FinSh& fs = sh.f;
  const int t = threadIdx.x, lane = t & (kWave - 1), wid = t / kWave;
  uint32_t prefix = 0, pmask = 0;
  uint64_t above = 0;
  for (int round = 0; round < 3; ++round) {
    const int shift = round == 0 ? 19 : (round == 1 ? 8 : 0);
    const uint32_t dmask = round == 0 ? 0xfffu : (round == 1 ? 0x7ffu : 0xffu);
    if (round > 0) {
#pragma unroll
      for (int q = 0; q < kBinsPerLane; ++q) fs.H[kBinsPerLane * t + q] = 0;
      __syncthreads();
    }
    visit([&](uint32_t bits, uint64_t w) {
      if ((bits & pmask) == prefix && w)
        __hip_atomic_fetch_add(&fs.H[digit_of(bits, shift, dmask)], w, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
    });
    __syncthreads();
    // lane t owns digits kBins-1 - (kBinsPerLane*t + q), q = 0.. (descending)
    uint64_t v[kBinsPerLane];
    uint64_t sum = 0;
#pragma unroll
    for (int q = 0; q < kBinsPerLane; ++q) {
      v[q] = fs.H[kBins - 1 - (kBinsPerLane * t + q)];
      sum += v[q];
    }
    uint64_t total;
    const uint64_t ex = block_excl_scan(sum, sh.red, &total);
    if (t == 0) sh.u32s[1] = kNone;
    __syncthreads();
    uint64_t before = above + ex;
    if (before < thr && before + sum >= thr) {
#pragma unroll
      for (int q = 0; q < kBinsPerLane; ++q) {
        if (before < thr && before + v[q] >= thr) {
          sh.u32s[1] = static_cast<uint32_t>(kBins - 1 - (kBinsPerLane * t + q));
          sh.u64s[1] = before;
          sh.u64s[2] = v[q];
        }
        before += v[q];
      }
    }
    if (t == 0) fs.gcount = 0;
    __syncthreads();
    const uint32_t digit = sh.u32s[1];
    if (digit == kNone) return false;
    prefix |= digit << shift;
    pmask |= dmask << shift;
    above = sh.u64s[1];
    const uint64_t binmass = sh.u64s[2];
    visit([&](uint32_t bits, uint64_t w) {
      if ((bits & pmask) == prefix && w) {
        const uint32_t k = __hip_atomic_fetch_add(&fs.gcount, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (k < kGather) {
          fs.gbits[k] = bits;
          fs.gw[k] = w;
        }
      }
    });
    __syncthreads();
    const uint32_t cnt = fs.gcount;
    if (cnt > kGather && round == 2) {
      // every entry of the bucket has the same bits
      *cutoff = __uint_as_float(prefix);
      *mass = above + binmass;
      return true;
    }
    if (cnt <= kGather) {
      if (wid == 0) {
        const uint32_t b = lane < static_cast<int>(cnt) ? fs.gbits[lane] : 0u;
        const uint64_t w = lane < static_cast<int>(cnt) ? fs.gw[lane] : 0;
        uint64_t A = above;
        for (int j = 0; j < static_cast<int>(cnt); ++j) {
          const uint32_t bj = lane_bcast_u32(b, j);
          const uint64_t wj = lane_bcast_u64(w, j);
          A += bj >= b ? wj : 0;
        }
        const bool ok = lane < static_cast<int>(cnt) && A >= thr;
        const uint64_t best = wave_max_u64(ok ? b : 0u);
        const uint64_t at = wave_max_u64(ok && b == static_cast<uint32_t>(best) ? A : 0);
        if (lane == 0) {
          sh.u32s[2] = static_cast<uint32_t>(best);
          sh.u64s[4] = at;
        }
      }
      __syncthreads();
      *cutoff = __uint_as_float(sh.u32s[2]);
      *mass = sh.u64s[4];
      return true;
    }
    __syncthreads();
  }
  return false;  // not reached
}

// p of element i of a row recomputed from its logit.
template <int DT>
__device__ __forceinline__ float p_elem(const char* rowp, const uint32_t* bm, float c, float pen, float inv_pen,
                                        const float* mcj, const float* gj, int i) {
  float l = load_elem<DT>(rowp, i);
  if (bm && bit_of(bm, i)) l = l < 0.0f ? l * pen : l * inv_pen;
  const int j = i >> kChunkShift;
  return exp2q(__builtin_fmaf(l, c, -mcj[j])) * gj[j];
}

// Index-ordered inverse-CDF pick over the first n LDS slots; weight(s) is an
// exact fx46 mass. Lane t owns slots [16t, 16t+16). Returns the winning slot,
// or -1 at zero total mass.
template <typename W>
__device__ int pick_slot(Shared& sh, int n, float u, W weight) {
  const int t = threadIdx.x;
  const int s0 = kSlotsPerLane * t;
  uint64_t sum = 0;
#pragma unroll
  for (int q = 0; q < kSlotsPerLane; ++q) sum += s0 + q < n ? weight(s0 + q) : 0;
  uint64_t total;
  const uint64_t ex = block_excl_scan(sum, sh.red, &total);
  if (t == 0) sh.u32s[3] = kNone;
  __syncthreads();
  if (total > 0) {
    const uint64_t target = floor_u_times(u, total);
    if (ex <= target && target < ex + sum) {
      uint64_t run = ex;
      for (int q = 0; q < kSlotsPerLane; ++q) {
        if (s0 + q >= n) break;
        run += weight(s0 + q);
        if (run > target) {
          sh.u32s[3] = static_cast<uint32_t>(s0 + q);
          break;
        }
      }
    }
  }
  __syncthreads();
  const uint32_t s = sh.u32s[3];
  return s == kNone ? -1 : static_cast<int>(s);
}

// Dense inverse-CDF pick over a whole row whose masses weight(idx) are
// computed on the fly. Lane t owns a contiguous index range.
template <typename W>
__device__ int64_t pick_dense(Shared& sh, int vocab, float u, W weight) {
  const int t = threadIdx.x;
  const int per = (vocab + kCB - 1) / kCB;
  const int a = t * per < vocab ? t * per : vocab;
  const int b = a + per < vocab ? a + per : vocab;
  uint64_t sum = 0;
  for (int i = a; i < b; ++i) sum += weight(i);
  uint64_t total;
  const uint64_t ex = block_excl_scan(sum, sh.red, &total);
  if (t == 0) sh.u64s[3] = 0;
  __syncthreads();
  if (total > 0) {
    const uint64_t target = floor_u_times(u, total);
    if (ex <= target && target < ex + sum) {
      uint64_t run = ex;
      for (int i = a; i < b; ++i) {
        run += weight(i);
        if (run > target) {
          sh.u64s[3] = static_cast<uint64_t>(i);
          break;
        }
      }
    }
  }
  __syncthreads();
  return static_cast<int64_t>(sh.u64s[3]);
}

// Exact select over every element of the row (the candidates did not hold the
// cutoff): p recomputed from the re-read logits, g_j in fs.g[0]. When keep is
// set, leaves the support {p >= c} in index order in fs.slot (as idx << 32 |
// bits(p)) and returns its size, or -1 if it does not fit. Out of line, with
// plain arguments, so the common path's registers are unaffected.
template <int DT>
__device__ __noinline__ int slow_select(Shared& sh, const char* rowp, const uint32_t* bm, float c, float pen,
                                        float inv_pen, int vocab, uint64_t thr, bool keep, float* cutoff,
                                        uint64_t* mass_fx) {
  FinSh& fs = sh.f;
  const int t = threadIdx.x;
  const float* mcj = fs.mcj[0];
  const float* gj = fs.g[0];
  auto pval = [&](int i) { return p_elem<DT>(rowp, bm, c, pen, inv_pen, mcj, gj, i); };
#pragma unroll
  for (int q = 0; q < kBinsPerLane; ++q) fs.H[kBinsPerLane * t + q] = 0;
  __syncthreads();
  float cc;
  uint64_t mfx;
  const bool ok = radix_select(sh, thr, [&](auto f) {
    for (int i = t; i < vocab; i += kCB) {
      const float pv = pval(i);
      f(__float_as_uint(pv), fx46(pv));
    }
  }, &cc, &mfx);
  if (!ok) {
    // Total mass below the threshold: keep the whole row (cutoff = min p).
    float mn = __builtin_inff();
    uint64_t tot = 0;
    for (int i = t; i < vocab; i += kCB) {
      const float pv = pval(i);
      mn = fminf(mn, pv);
      tot += fx46(pv);
    }
    mn = wave_max_f32(-mn);
    if ((t & (kWave - 1)) == 0) sh.f32s[t / kWave] = mn;
    tot = block_sum(tot, sh.red);
    cc = -nmax(nmax(sh.f32s[0], sh.f32s[1]), nmax(sh.f32s[2], sh.f32s[3]));
    mfx = tot;
    __syncthreads();
  }
  *cutoff = cc;
  *mass_fx = mfx;
  if (!keep) return -1;
  const int per = (vocab + kCB - 1) / kCB;
  const int a = t * per < vocab ? t * per : vocab;
  const int b = a + per < vocab ? a + per : vocab;
  uint64_t cnt = 0;
  for (int i = a; i < b; ++i) cnt += pval(i) >= cc ? 1 : 0;
  uint64_t total;
  const uint64_t ex = block_excl_scan(cnt, sh.red, &total);
  if (total > static_cast<uint64_t>(kRowCand)) return -1;
  int pos = static_cast<int>(ex);
  for (int i = a; i < b; ++i) {
    const float pv = pval(i);
    if (pv >= cc) fs.slot[pos++] = (static_cast<uint64_t>(i) << 32) | __float_as_uint(pv);
  }
  __syncthreads();
  return static_cast<int>(total);
}

// Candidate slot s of row r: (idx << 32 | bits(e)); stale beyond n_j.
__device__ __forceinline__ uint64_t load_slot(const SampParams& p, int64_t r, int s) {
  return p.cands[(r * p.nch + (s >> p.cap_log2)) * kChunkCand + (s & (p.cap - 1))];
}

__device__ __forceinline__ bool slot_valid(const FinSh& fs, int slot, const SampParams& p, int s) {
  return (s & (p.cap - 1)) < static_cast<int>(fs.n[slot][s >> p.cap_log2]);
}

// Inverse-CDF draw over this workgroup's own row (fs.slot holds idx | bits(p)
// of n slots, fs.g[0] / fs.mcj[0] the row's scales): weights fx46(P), P the
// filtered, renormalised probability; the whole row when it is dense.
template <int DT>
__device__ int64_t own_draw(const SampParams& p, Shared& sh, const RowStat& st, int n, float u, const char* rowp,
                            const uint32_t* bm) {
  FinSh& fs = sh.f;
  const bool unf = st.flags & kFlagUnfiltered;
  if (!(st.flags & kFlagDense)) {
    const float cc = st.cutoff, mass = st.mass;
    const int win = pick_slot(sh, n, u, [&](int s) {
      const float x = __uint_as_float(static_cast<uint32_t>(fs.slot[s]));
      return x >= cc && x > 0.0f ? fx46(x / mass) : 0ull;
    });
    return win < 0 ? 0 : static_cast<int64_t>(fs.slot[win] >> 32);
  }
  const float cc = st.cutoff, mass = st.mass;
  return pick_dense(sh, p.vocab, u, [&](int i) {
    const float x = p_elem<DT>(rowp, bm, p.c, p.pen, p.inv_pen, fs.mcj[0], fs.g[0], i);
    return fx46(unf ? x : (x >= cc ? x / mass : 0.0f));
  });
}

// Residual draw for draft position i of group g: normalize(max(P_i - Q_i, 0))
// (fallback normalize(P_i), rejection.py:60-69) with the uniform u[g, k+i].
// P_i comes from the target row's candidates (already in fs.slot / fs.g[0]
// when `own`, i.e. this workgroup finalised the target row); Q_i is
// recomputed from the draft logits at the support indices.
template <int DT>
__device__ int64_t residual_draw(const SampParams& p, Shared& sh, int64_t g, int i, bool own) {
  FinSh& fs = sh.f;
  const int k = p.k, rpg = 2 * k + 1, nch = p.nch, nslots = nch * p.cap;
  const int t = threadIdx.x, wid = t / kWave;
  const int64_t rt = g * rpg + i, rd = g * rpg + k + 1 + i;
  // 1. both rows' statistics, chunk records, and the target's candidates
  if (t < 8) fs.statw[t] = load_sc64(reinterpret_cast<const uint64_t*>(p.stats + (t < 4 ? rt : rd)) + (t & 3));
  ChunkRec rt_a{}, rt_b{}, rd_a{}, rd_b{};
  if (wid == 0) {
    load_recs(p, rd, &rd_a, &rd_b);
    if (!own) load_recs(p, rt, &rt_a, &rt_b);
  }
  if (!own) {
#pragma unroll
    for (int q = 0; q < kSlotsPerLane; ++q) {
      const int s = t + q * kCB;
      if (s < nslots) fs.slot[s] = load_slot(p, rt, s);
    }
  }
  __syncthreads();
  const RowStat st_t = stat_of(fs.statw[0], fs.statw[1], fs.statw[2], fs.statw[3]);
  const RowStat st_d = stat_of(fs.statw[4], fs.statw[5], fs.statw[6], fs.statw[7]);
  if (wid == 0) {
    if (!own) row_g(fs, 0, rt_a, rt_b, nch, st_t.mcmax, st_t.s);
    row_g(fs, 1, rd_a, rd_b, nch, st_d.mcmax, st_d.s);
  }
  __syncthreads();
  const bool unf_t = st_t.flags & kFlagUnfiltered;
  const bool unf_d = st_d.flags & kFlagUnfiltered;
  const float u = p.uniforms[g * rpg + k + i];
  const uint32_t* bm = p.use_pen ? p.bitmap + g * p.bm_words : nullptr;
  const char* drow = row_of(p, g, k + 1 + i);
  auto Qof = [&](float l, int j) {
    const float x = exp2q(__builtin_fmaf(l, p.c, -fs.mcj[1][j])) * fs.g[1][j];
    return unf_d ? x : (x >= st_d.cutoff ? x / st_d.mass : 0.0f);
  };
  if (!(st_t.flags & kFlagDense)) {
    // P over the target's support, the draft logits there gathered at once
    float P[kSlotsPerLane], lq[kSlotsPerLane];
#pragma unroll
    for (int q = 0; q < kSlotsPerLane; ++q) {
      const int s = t + q * kCB;
      P[q] = 0.0f;
      lq[q] = 0.0f;
      if (s < nslots && slot_valid(fs, 0, p, s)) {
        const uint64_t v = fs.slot[s];
        const float pv = own ? __uint_as_float(static_cast<uint32_t>(v))
                             : __uint_as_float(static_cast<uint32_t>(v)) * fs.g[0][s >> p.cap_log2];
        if (pv >= st_t.cutoff && pv > 0.0f) {
          P[q] = pv / st_t.mass;
          lq[q] = load_elem<DT>(drow, static_cast<int64_t>(v >> 32));
        }
      }
    }
    float D[kSlotsPerLane];
    uint64_t dsum = 0, psum = 0;
#pragma unroll
    for (int q = 0; q < kSlotsPerLane; ++q) {
      const int s = t + q * kCB;
      D[q] = 0.0f;
      if (P[q] > 0.0f) {
        const int idx = static_cast<int>(fs.slot[s] >> 32);
        float l = lq[q];
        if (bm && bit_of(bm, idx)) l = l < 0.0f ? l * p.pen : l * p.inv_pen;
        const float dv = P[q] - Qof(l, idx >> kChunkShift);
        D[q] = dv > 0.0f ? dv : 0.0f;
        dsum += fx46(D[q]);
        psum += fx46(P[q]);
      }
    }
    const uint64_t d_fx = block_sum(dsum, sh.red);
    const uint64_t p_fx = block_sum(psum, sh.red);
    const bool use_d = d_fx > 0;
    const float den = use_d ? mass_to_f32(d_fx) : (p_fx > 0 ? mass_to_f32(p_fx) : 1.0f);
#pragma unroll
    for (int q = 0; q < kSlotsPerLane; ++q) {
      const int s = t + q * kCB;
      if (s < nslots) fs.w[s] = (use_d ? D[q] : P[q]) / den;
    }
    __syncthreads();
    const int win = pick_slot(sh, nslots, u, [&](int s) { return fx46(fs.w[s]); });
    return win < 0 ? 0 : static_cast<int64_t>(fs.slot[win] >> 32);
  }
  // dense target row: the whole vocabulary
  const char* trow = row_of(p, g, i);
  auto Pof = [&](int x) {
    const float pv = p_elem<DT>(trow, bm, p.c, p.pen, p.inv_pen, fs.mcj[0], fs.g[0], x);
    return unf_t ? pv : (pv >= st_t.cutoff ? pv / st_t.mass : 0.0f);
  };
  auto Qat = [&](int x) {
    float l = load_elem<DT>(drow, x);
    if (bm && bit_of(bm, x)) l = l < 0.0f ? l * p.pen : l * p.inv_pen;
    return Qof(l, x >> kChunkShift);
  };
  uint64_t dsum = 0, psum = 0;
  {
    const int per = (p.vocab + kCB - 1) / kCB;
    const int i0 = t * per < p.vocab ? t * per : p.vocab;
    const int i1 = i0 + per < p.vocab ? i0 + per : p.vocab;
    for (int x = i0; x < i1; ++x) {
      const float pj = Pof(x);
      const float dj = pj - Qat(x);
      dsum += fx46(dj > 0.0f ? dj : 0.0f);
      psum += fx46(pj);
    }
  }
  const uint64_t d_fx = block_sum(dsum, sh.red);
  const uint64_t p_fx = block_sum(psum, sh.red);
  const bool use_d = d_fx > 0;
  const float den = use_d ? mass_to_f32(d_fx) : (p_fx > 0 ? mass_to_f32(p_fx) : 1.0f);
  return pick_dense(sh, p.vocab, u, [&](int x) {
    const float pj = Pof(x);
    float v = pj;
    if (use_d) {
      const float dj = pj - Qat(x);
      v = dj > 0.0f ? dj : 0.0f;
    }
    return fx46(v / den);
  });
}

// The accept chain of group g once every draw is published: the first
// rejected position a (u < min(1, P/Q) per position, sampler.py:451-452),
// then the accepted drafts, the draw of position a, and -1 after it.
__device__ void accept_chain(const SampParams& p, Shared& sh, int64_t g) {
  FinSh& fs = sh.f;
  const int k = p.k, rpg = 2 * k + 1;
  const int t = threadIdx.x, lane = t & (kWave - 1), wid = t / kWave;
  const int64_t r0 = g * rpg;
  if (t < rpg) fs.tokp[t] = hi_f(load_sc64(reinterpret_cast<const uint64_t*>(p.stats + r0 + t) + 2));
  if (t <= k) fs.tokd[t] = static_cast<int64_t>(load_sc64(reinterpret_cast<const uint64_t*>(p.draws) + g * (k + 1) + t));
  int64_t x = -1;
  float ux = 0.0f;
  if (wid == 0 && lane < k) {
    x = p.draft_tokens[g * k + lane];
    ux = p.uniforms[g * rpg + lane];
  }
  __syncthreads();
  if (wid == 0) {
    const bool valid = x >= 0 && x < p.vocab;
    const bool ok = lane < k && valid && accept_draw(ux, fs.tokp[lane], fs.tokp[k + 1 + lane]);
    const uint64_t bad = __ballot(lane < k && !ok);
    const int a = bad ? __builtin_ctzll(bad) : k;
    int64_t* out = p.tokens + g * (k + 1);
    if (lane < a) out[lane] = x;
    if (lane == a) out[lane] = fs.tokd[a];
    if (lane > a && lane <= k) out[lane] = -1;
    if (k >= kWave && lane == 0) {
      for (int j = kWave; j <= k; ++j) out[j] = j < a ? p.draft_tokens[g * k + j] : (j == a ? fs.tokd[a] : -1);
    }
    if (lane == 0) p.accept_len[g] = a;
  }
}

// Row finalisation: one workgroup per row.
template <int DT, int MODE>
__global__ __launch_bounds__(kCB) void row_kernel(const SampParams p) {
  __shared__ Shared sh;
  FinSh& fs = sh.f;
  const int r = blockIdx.x;
  const int t = threadIdx.x, wid = t / kWave;
  const int nch = p.nch;
  const int64_t g = r / p.rpg;
  const int jr = r - static_cast<int>(g) * p.rpg;
  const int nslots = nch * p.cap;
  const float top_p = p.top_p_rows ? p.top_p_rows[r] : p.top_p;
  const bool unfiltered = !(top_p < 1.0f);
  const char* rowp = row_of(p, g, jr);
  const uint32_t* bm = p.use_pen ? p.bitmap + g * p.bm_words : nullptr;

  // 1. chunk records (wave 0) and candidate slots (strided), in flight together
  ChunkRec ra{}, rb{};
  if (wid == 0) load_recs(p, r, &ra, &rb);
  uint64_t cv[kSlotsPerLane];
#pragma unroll
  for (int q = 0; q < kSlotsPerLane; ++q) {
    const int s = t + q * kCB;
    cv[q] = (!unfiltered && s < nslots) ? load_slot(p, r, s) : 0;
  }
#pragma unroll
  for (int q = 0; q < kBinsPerLane; ++q) fs.H[kBinsPerLane * t + q] = 0;
  // 2. row scales
  if (wid == 0) {
    const RowScale rs = row_scale(fs, 0, ra, rb, nch);
    if (t == 0) {
      sh.f32s[4] = rs.mcmax;
      sh.f32s[5] = rs.s;
      sh.f32s[6] = rs.p_bound;
      sh.f32s[7] = rs.has_tok ? rs.p_tok : -1.0f;
    }
  }
  __syncthreads();
  const float mcmax = sh.f32s[4], s_row = sh.f32s[5], p_bound = sh.f32s[6], p_tok = sh.f32s[7];
  // 3. p of the candidates, kept in registers and in fs.slot
  float pv[kSlotsPerLane];
#pragma unroll
  for (int q = 0; q < kSlotsPerLane; ++q) {
    const int s = t + q * kCB;
    pv[q] = 0.0f;
    if (!unfiltered && s < nslots && slot_valid(fs, 0, p, s))
      pv[q] = __uint_as_float(static_cast<uint32_t>(cv[q])) * fs.g[0][s >> p.cap_log2];
    if (s < nslots) fs.slot[s] = ((cv[q] >> 32) << 32) | __float_as_uint(pv[q]);
  }
  float cutoff = 0.0f;
  uint64_t mass_fx = 0;
  uint32_t flags = unfiltered ? (kFlagUnfiltered | kFlagDense) : 0u;
  int n_sup = nslots;
  if (!unfiltered) {
    const uint64_t thr = fx46(top_p);
    float c;
    uint64_t mfx;
    const bool ok = radix_select(sh, thr, [&](auto f) {
#pragma unroll
      for (int q = 0; q < kSlotsPerLane; ++q) {
        const float x = pv[q];
        if (x > 0.0f) f(__float_as_uint(x), fx46(x));
      }
    }, &c, &mfx);
    if (ok && c > p_bound) {
      cutoff = c;
      mass_fx = mfx;
    } else {
      flags |= kFlagSlow;
      __syncthreads();
      n_sup = slow_select<DT>(sh, rowp, bm, p.c, p.pen, p.inv_pen, p.vocab, thr, MODE == kModeSample, &cutoff,
                              &mass_fx);
      if (MODE != kModeSample || n_sup < 0) flags |= kFlagDense;
    }
  }
  RowStat st;
  st.mcmax = mcmax;
  st.s = s_row;
  st.cutoff = cutoff;
  st.mass = unfiltered ? 1.0f : mass_to_f32(mass_fx);
  st.flags = flags;
  st.p_tok = 0.0f;
  st.mass_fx = mass_fx;
  if (p_tok >= 0.0f) st.p_tok = unfiltered ? p_tok : (p_tok >= cutoff ? p_tok / st.mass : 0.0f);

  if constexpr (MODE == kModeSpec) {
    const int k = p.k;
    if (t == 0) {
      put_stat(p.stats + r, st);
      drain_stores();
    }
    // Pair (target i, draft i): the second to finish draws position i's
    // residual; the bonus row draws the bonus token. Each draw arrives on the
    // group's counter; the last arrival runs the accept chain.
    bool draw_here = jr == k;
    const int i = jr < k ? jr : jr - k - 1;
    if (jr != k) {
      if (t == 0) {
        uint32_t* ctr = p.row_cnt + (g * p.rpg + i) * kCounterStride;
        const uint32_t prev = atomic_arrive(ctr);
        if (prev == 1u) store_sc(ctr, 0u);
        sh.u32s[6] = prev == 1u ? 1u : 0u;
      }
      __syncthreads();
      draw_here = sh.u32s[6] != 0u;
    }
    if (draw_here) {
      const int64_t tok = jr == k ? own_draw<DT>(p, sh, st, nslots, p.uniforms[g * p.rpg + 2 * k], rowp, bm)
                                  : residual_draw<DT>(p, sh, g, i, jr < k);
      if (t == 0) {
        store_sc64(reinterpret_cast<uint64_t*>(p.draws) + g * (k + 1) + (jr == k ? k : i), static_cast<uint64_t>(tok));
        drain_stores();
        uint32_t* ctr = p.grp_cnt + g * kCounterStride;
        const uint32_t prev = atomic_arrive(ctr);
        const bool last = prev == static_cast<uint32_t>(k);
        if (last) store_sc(ctr, 0u);
        sh.u32s[7] = last ? 1u : 0u;
      }
      __syncthreads();
      if (sh.u32s[7]) accept_chain(p, sh, g);
    }
  } else if constexpr (MODE == kModeSample) {
    const int64_t token = own_draw<DT>(p, sh, st, (flags & kFlagSlow) ? n_sup : nslots, p.row_uniforms[r], rowp, bm);
    if (t == 0) p.row_tokens[r] = token;
  } else {
    if (t == 0) {
      p.stats[r] = st;
      if (p.cutoff_out) p.cutoff_out[r] = unfiltered ? 0.0f : cutoff;
      if (p.mass_out) p.mass_out[r] = st.mass;
    }
  }
}

// ===========================================================================
// dense_kernel: p and the filtered distribution for one (row, chunk) item
// ===========================================================================
template <int DT>
__global__ __launch_bounds__(kCB) void dense_kernel(const SampParams p) {
  constexpr int EPV = Elem<DT>::kPerVec;
  constexpr int NVC = kChunk / (kCB * EPV);
  const int t = threadIdx.x;
  const int item = blockIdx.x;
  const int64_t r = item / p.nch;
  const int cj = item - static_cast<int>(r) * p.nch;
  const char* rowp = row_of(p, r, 0);
  const int c0 = cj * kChunk;
  const int nel = p.vocab - c0 < kChunk ? p.vocab - c0 : kChunk;
  const int nvc = nel / EPV;
  const u32x4* src = reinterpret_cast<const u32x4*>(rowp) + c0 / EPV;
  const RowStat st = p.stats[r];
  const float mc = p.chunks[r * p.nch + cj].mc;
  const float gj = exp2q(mc - st.mcmax) / st.s;
  const bool unf = st.flags & kFlagUnfiltered;
#pragma unroll
  for (int u = 0; u < NVC; ++u) {
    const int v = u * kCB + t;
    if (v < nvc) {
      const u32x4 d = __builtin_nontemporal_load(src + v);
      float pv[EPV], fv[EPV];
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        const float x = exp2q(__builtin_fmaf(vec_elem<DT>(d, e), p.c, -mc)) * gj;
        pv[e] = x;
        fv[e] = unf ? x : (x >= st.cutoff ? x / st.mass : 0.0f);
      }
      const int64_t i = c0 + static_cast<int64_t>(v) * EPV;
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        if (p.probs_out) p.probs_out[r * p.probs_stride + i + e] = pv[e];
        if (p.filt_out) p.filt_out[r * p.filt_stride + i + e] = fv[e];
      }
    }
  }
}

// ===========================================================================
// Host side
// ===========================================================================
struct Layout {
  uint64_t row_cnt, grp_cnt, chunks, cands, stats, draws, bitmap, total;
};

// Workspace: [pair arrival counters, one 64-byte line each, for up to
// kMaxRows rows] [group counters for up to kMaxSpecBatch elements] (both at
// fixed places, so calls of any shape find them zero) [chunk records]
// [candidates] [row statistics] [draws] [penalty bitmaps, one per group].
Layout ws_layout(int64_t rows, int64_t groups, int nch) {
  auto al = [](uint64_t x) { return (x + 255u) & ~255ull; };
  Layout l{};
  l.row_cnt = 0;
  l.grp_cnt = al(static_cast<uint64_t>(kMaxRows) * kCounterStride * 4u);
  uint64_t off = al(l.grp_cnt + static_cast<uint64_t>(kMaxSpecBatch) * kCounterStride * 4u);
  l.chunks = off;
  off = al(off + static_cast<uint64_t>(rows) * nch * sizeof(ChunkRec));
  l.cands = off;
  off = al(off + static_cast<uint64_t>(rows) * nch * kChunkCand * 8u);
  l.stats = off;
  off = al(off + static_cast<uint64_t>(rows) * sizeof(RowStat));
  l.draws = off;
  off = al(off + static_cast<uint64_t>(rows) * 8u);
  l.bitmap = off;
  off = al(off + static_cast<uint64_t>(groups) * nch * (kChunk / 32) * 4u);
  l.total = off;
  return l;
}

void bind_workspace(SampParams& p, void* ws, const Layout& l) {
  char* b = static_cast<char*>(ws);
  p.row_cnt = reinterpret_cast<uint32_t*>(b + l.row_cnt);
  p.grp_cnt = reinterpret_cast<uint32_t*>(b + l.grp_cnt);
  p.chunks = reinterpret_cast<ChunkRec*>(b + l.chunks);
  p.cands = reinterpret_cast<uint64_t*>(b + l.cands);
  p.stats = reinterpret_cast<RowStat*>(b + l.stats);
  p.draws = reinterpret_cast<int64_t*>(b + l.draws);
  p.bitmap = reinterpret_cast<uint32_t*>(b + l.bitmap);
}

int nch_for(int64_t vocab) { return static_cast<int>((vocab + kChunk - 1) / kChunk); }

template <int DT, int MODE>
void launch_dt(const SampParams& p, int64_t groups, int64_t rows, hipStream_t st) {
  if (p.use_pen) hipLaunchKernelGGL(bitmap_kernel, dim3(static_cast<unsigned>(groups)), dim3(kBmB), 0, st, p);
  const int wgs = static_cast<int>(device_cu_count()) * kChunkWavesPerCu;
  hipLaunchKernelGGL((chunk_kernel<DT>), dim3(p.items < wgs ? p.items : wgs), dim3(kWave), 0, st, p);
  hipLaunchKernelGGL((row_kernel<DT, MODE>), dim3(static_cast<unsigned>(rows)), dim3(kCB), 0, st, p);
  if constexpr (MODE == kModeDense) {
    hipLaunchKernelGGL((dense_kernel<DT>), dim3(p.items), dim3(kCB), 0, st, p);
  }
}

template <int MODE>
int launch_mode(const SampParams& p, int dtype, int64_t groups, int64_t rows, hipStream_t st) {
  switch (dtype) {
    case LS_DTYPE_F32: launch_dt<F32, MODE>(p, groups, rows, st); break;
    case LS_DTYPE_BF16: launch_dt<BF16, MODE>(p, groups, rows, st); break;
    case LS_DTYPE_F16: launch_dt<F16, MODE>(p, groups, rows, st); break;
    default: return fail(LS_ERR_VALUE, "unsupported logits dtype");
  }
  return check_launch("sampling kernel launch");
}

// Shared argument validation / setup for the processing options.
int setup_common(SampParams& p, int dtype, int64_t rows, int64_t vocab, float temperature, float top_p,
                 int64_t top_k, float penalty, const int32_t* history, int64_t history_stride,
                 const int32_t* history_len) {
  const int eb = dtype_bytes(dtype);
  if (eb == 0) return fail(LS_ERR_VALUE, "unsupported logits dtype");
  if (vocab <= 0 || vocab > kMaxVocab) return fail(LS_ERR_VALUE, "vocabulary size must be in [1, 262144]");
  if ((vocab * eb) % 16 != 0) return fail(LS_ERR_VALUE, "vocabulary row bytes must be a multiple of 16");
  if (rows > kMaxRows) return fail(LS_ERR_VALUE, "at most 65536 logit rows per call");
  if (!(temperature > 0.0f)) return fail(LS_ERR_VALUE, "temperature must be > 0");
  if (!(top_p > 0.0f) || top_p > 1.0f) return fail(LS_ERR_VALUE, "top_p must be in (0, 1]");
  if (top_k != 0 && top_k < vocab) return fail(LS_ERR_VALUE, "top_k filtering is not supported by this entry point");
  if (!(penalty > 0.0f)) return fail(LS_ERR_VALUE, "repetition penalty must be > 0");
  if (penalty != 1.0f && (history == nullptr || history_len == nullptr))
    return fail(LS_ERR_VALUE, "repetition penalty needs a token history");
  p.vocab = static_cast<int>(vocab);
  p.nch = nch_for(vocab);
  p.cap_log2 = p.nch <= kRowCand / kChunkCand ? 6 : (p.nch <= 2 * kRowCand / kChunkCand ? 5 : 4);
  p.cap = 1 << p.cap_log2;  // nch * cap <= kRowCand
  p.bm_words = p.nch * (kChunk / 32);
  p.items = static_cast<int>(rows * p.nch);
  const float inv_t = 1.0f / temperature;
  p.c = kLog2e * inv_t;
  p.use_pen = penalty != 1.0f;
  p.pen = penalty;
  p.inv_pen = 1.0f / penalty;
  p.top_p = top_p;
  p.hist = history;
  p.hist_stride = history_stride;
  p.hist_len = history_len;
  return LS_OK;
}

}  // namespace
}  // namespace ls

using namespace ls;

extern "C" {

uint64_t ls_spec_verify_workspace(int64_t batch, int64_t k, int64_t vocab) {
  if (batch <= 0 || k < 1 || vocab <= 0) return 0;
  return ws_layout(batch * (2 * k + 1), batch, nch_for(vocab)).total;
}

int ls_spec_verify(const void* target_logits, int64_t target_batch_stride, int64_t target_pos_stride,
                   const void* draft_logits, int64_t draft_batch_stride, int64_t draft_pos_stride,
                   const int64_t* draft_tokens, const float* uniforms, int dtype, int64_t batch, int64_t k,
                   int64_t vocab, float temperature, float top_p, int64_t top_k, float penalty,
                   const int32_t* history, int64_t history_stride, const int32_t* history_len,
                   int32_t* accept_len, int64_t* tokens, void* workspace, uint64_t ws_bytes, ls_stream_t stream) {
  if (batch < 0 || batch > kMaxSpecBatch || k < 1 || k > 64)
    return fail(LS_ERR_VALUE, "spec_verify: need 0 <= batch <= 16384 and 1 <= k <= 64");
  if (batch == 0) return LS_OK;
  if (!target_logits || !draft_logits || !draft_tokens || !uniforms || !accept_len || !tokens)
    return fail(LS_ERR_VALUE, "spec_verify: NULL pointer");
  SampParams p{};
  const int64_t rows = batch * (2 * k + 1);
  int rc = setup_common(p, dtype, rows, vocab, temperature, top_p, top_k, penalty, history, history_stride,
                        history_len);
  if (rc) return rc;
  const int eb = dtype_bytes(dtype);
  p.base0 = static_cast<const char*>(target_logits);
  p.bstride0 = target_batch_stride * eb;
  p.pstride0 = target_pos_stride * eb;
  p.base1 = static_cast<const char*>(draft_logits);
  p.bstride1 = draft_batch_stride * eb;
  p.pstride1 = draft_pos_stride * eb;
  if (!aligned16(target_logits) || !aligned16(draft_logits) || p.bstride0 % 16 || p.pstride0 % 16 ||
      p.bstride1 % 16 || p.pstride1 % 16)
    return fail(LS_ERR_VALUE, "spec_verify: logits rows must be 16-byte aligned");
  p.k = static_cast<int>(k);
  p.rpg = static_cast<int>(2 * k + 1);
  p.draft_tokens = draft_tokens;
  p.uniforms = uniforms;
  p.accept_len = accept_len;
  p.tokens = tokens;
  const Layout l = ws_layout(rows, batch, p.nch);
  if (!workspace || ws_bytes < l.total) return fail(LS_ERR_VALUE, "spec_verify: workspace too small");
  bind_workspace(p, workspace, l);
  return launch_mode<kModeSpec>(p, dtype, batch, rows, static_cast<hipStream_t>(stream));
}

uint64_t ls_sample_logits_workspace(int64_t rows, int64_t vocab) {
  if (rows <= 0 || vocab <= 0) return 0;
  return ws_layout(rows, rows, nch_for(vocab)).total;
}

int ls_sample_logits(const void* logits, int64_t row_stride, int dtype, int64_t rows, int64_t vocab,
                     float temperature, float top_p, int64_t top_k, float penalty, const int32_t* history,
                     int64_t history_stride, const int32_t* history_len, const float* uniforms,
                     int64_t* out_tokens, void* workspace, uint64_t ws_bytes, ls_stream_t stream) {
  if (rows < 0 || rows > kMaxRows) return fail(LS_ERR_VALUE, "sample_logits: need 0 <= rows <= 65536");
  if (rows == 0) return LS_OK;
  if (!logits || !uniforms || !out_tokens) return fail(LS_ERR_VALUE, "sample_logits: NULL pointer");
  SampParams p{};
  int rc = setup_common(p, dtype, rows, vocab, temperature, top_p, top_k, penalty, history, history_stride,
                        history_len);
  if (rc) return rc;
  const int eb = dtype_bytes(dtype);
  p.base0 = static_cast<const char*>(logits);
  p.bstride0 = row_stride * eb;
  if (!aligned16(logits) || p.bstride0 % 16) return fail(LS_ERR_VALUE, "sample_logits: rows must be 16-byte aligned");
  p.rpg = 1;
  p.k = 0;
  p.row_uniforms = uniforms;
  p.row_tokens = out_tokens;
  const Layout l = ws_layout(rows, rows, p.nch);
  if (!workspace || ws_bytes < l.total) return fail(LS_ERR_VALUE, "sample_logits: workspace too small");
  bind_workspace(p, workspace, l);
  return launch_mode<kModeSample>(p, dtype, rows, rows, static_cast<hipStream_t>(stream));
}

uint64_t ls_filter_logits_workspace(int64_t rows, int64_t vocab) {
  if (rows <= 0 || vocab <= 0) return 0;
  return ws_layout(rows, rows, nch_for(vocab)).total;
}

int ls_filter_logits(const void* logits, int64_t row_stride, int dtype, int64_t rows, int64_t vocab,
                     float temperature, float top_p, const float* top_p_rows, int64_t top_k, float* probs_out,
                     int64_t probs_stride, float* filtered_out, int64_t filtered_stride, float* cutoff_out,
                     float* mass_out, void* workspace, uint64_t ws_bytes, ls_stream_t stream) {
  if (rows < 0 || rows > kMaxRows) return fail(LS_ERR_VALUE, "filter_logits: need 0 <= rows <= 65536");
  if (rows == 0) return LS_OK;
  if (!logits) return fail(LS_ERR_VALUE, "filter_logits: NULL logits");
  SampParams p{};
  int rc = setup_common(p, dtype, rows, vocab, temperature, top_p, top_k, 1.0f, nullptr, 0, nullptr);
  if (rc) return rc;
  const int eb = dtype_bytes(dtype);
  p.base0 = static_cast<const char*>(logits);
  p.bstride0 = row_stride * eb;
  if (!aligned16(logits) || p.bstride0 % 16) return fail(LS_ERR_VALUE, "filter_logits: rows must be 16-byte aligned");
  p.rpg = 1;
  p.k = 0;
  p.top_p_rows = top_p < 1.0f ? top_p_rows : nullptr;
  p.probs_out = probs_out;
  p.probs_stride = probs_stride;
  p.filt_out = filtered_out;
  p.filt_stride = filtered_stride;
  p.cutoff_out = cutoff_out;
  p.mass_out = mass_out;
  const Layout l = ws_layout(rows, rows, p.nch);
  if (!workspace || ws_bytes < l.total) return fail(LS_ERR_VALUE, "filter_logits: workspace too small");
  bind_workspace(p, workspace, l);
  return launch_mode<kModeDense>(p, dtype, rows, rows, static_cast<hipStream_t>(stream));
}

}  // extern "C"
