// (a) logit processing and (c) lossless speculative sampling for gfx950.
//
// Two launches per call (a third, first, with a repetition penalty; a last
// one for dense outputs):
//   bitmap_kernel    one workgroup per batch element turns its token history
//                    into a vocabulary bitmap in the workspace.
//   chunk_kernel     persistent, one wave per (row, chunk) item of kChunk =
//                    2048 logits, items in row-major order, the next item's
//                    loads in flight while the current one is processed. Per
//                    item: the penalised chunk max m_j, mc_j = RN(m_j c) with
//                    c = RN(log2e RN(1/T)), e = exp2q(fma(x, c, -mc_j)), the
//                    chunk mass M_j (a fixed pairwise tree), a histogram of
//                    exp2q's exponent (bins 0..15 below the chunk max) and the
//                    chunk's candidates: every e >= kCandScale 2^-K, K the
//                    number of leading bins holding at most cap entries
//                    together, written in index order; then a 32-byte record
//                    (mc_j, K, count, M_j, e of the row's draft token).
//   spec_row_kernel  one 512-lane workgroup per (batch element, position i):
//                    the target and the draft row of position i side by side
//                    (the bonus row alone for i == k). S = sum_j f_j M_j with
//                    f_j = exp2q(mc_j - max mc), g_j = RN(f_j / S),
//                    p = RN(e g_j) for the candidates; the exact top-p cutoff
//                    by a radix select on the binary32 bits of p with 2^-46
//                    fixed-point masses (replacing sort + cumsum +
//                    searchsorted, distributions.py:59-70), valid iff it
//                    exceeds the bound on every p outside the candidates
//                    (otherwise the row is re-read for an exact select); the
//                    accept bit of x_i and the residual draw. The last of the
//                    k+1 workgroups of a batch element writes its accepted
//                    length and tokens.
//   row_kernel       sample and dense modes: one workgroup per row, the same
//                    finalisation, then a draw or the row statistics.
//   dense_kernel     dense mode: p and/or the filtered, renormalised rows.
// The arithmetic is the declared arithmetic of ls_numerics.hpp (restated by
// oracle/sampling.py), so every output is bit-identical to the oracle's.
#include "ls_common.hpp"
#include "ls_numerics.hpp"
#include "ls_runtime.hpp"

namespace ls {
namespace {

constexpr int kChunk = 2048;                 // softmax chunk (declared arithmetic)
constexpr int kChunkShift = 11;
constexpr int kCB = 256;                     // dense kernel lanes
constexpr int kRB = 512;                     // row kernel lanes
constexpr int kRW = kRB / kWave;
constexpr int kPerLane = kChunk / kWave;     // 32 elements per lane: one wave per chunk
constexpr int kChunkCand = 64;               // candidate slots per chunk in the workspace
constexpr int kOctBins = 16;                 // exponent bins of e
constexpr int kHistStride = kOctBins + 1;    // bins of a lane pair, padded against bank conflicts
constexpr int kHistRows = kWave / 2;         // lanes t and t + 32 share a row of bins
constexpr int kRowCand = 2048;               // candidate slots of a row
constexpr int kSlotsPerLane = kRowCand / kRB;
constexpr int kMaxChunks = 128;              // vocab <= 262144
constexpr int kMaxVocab = kMaxChunks * kChunk;
constexpr int kBins = 2048;                  // radix digits per round
constexpr int kBinsPerLane = kBins / kRB;
constexpr int kGather = kWave;               // bucket size finished by one wave
constexpr int kCounterStride = 16;           // arrival counters one 64-byte line apart
// Resident chunk waves per CU: 15 fit the LDS, but 12 measured fastest on
// MI355X (C3 and C4: 8, 10 and 15 all slower).
constexpr int kChunkWavesPerCu = 12;
constexpr int64_t kMaxRows = 65536;
constexpr int64_t kMaxSpecBatch = 16384;
constexpr uint32_t kNone = 0xffffffffu;

enum Mode : int { kModeSpec = 0, kModeSample = 1, kModeDense = 2 };
// kFlagRebuilt: the candidates of some chunks were replaced (same slot layout)
enum RowFlag : uint32_t { kFlagUnfiltered = 1u, kFlagDense = 2u, kFlagSlow = 4u, kFlagRebuilt = 8u };
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
  // exponent bins, 16-bit counts: lane t < 32 counts bin b in the low half of
  // word b of row t, lane t + 32 in the high half of word 15 - b of row t
  // (the two lanes meet on one word only for bins 0 and 15, rarely together)
  uint32_t hist[kHistRows * kHistStride];
};

// Physical float index of element v of the chunk in the e-store.
__device__ __forceinline__ int est_index(int v) {
  const int s = v >> 2;
  return ((s ^ ((s >> 3) & 7)) << 2) | (v & 3);
}

__device__ __forceinline__ uint64_t pack2(uint32_t lo, uint32_t hi) {
  return static_cast<uint64_t>(lo) | (static_cast<uint64_t>(hi) << 32);
}
__device__ __forceinline__ uint64_t pack2f(float lo, float hi) { return pack2(__float_as_uint(lo), __float_as_uint(hi)); }
__device__ __forceinline__ float lo_f(uint64_t v) { return __uint_as_float(static_cast<uint32_t>(v)); }
__device__ __forceinline__ float hi_f(uint64_t v) { return __uint_as_float(static_cast<uint32_t>(v >> 32)); }

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

// Bins and candidates: bin b = min(-k, 15) counts the elements whose
// exponent scaling in exp2q is 2^k = 2^-b (e in [2^-b / sqrt2, 2^-b * sqrt2)),
// the last bin also everything smaller; lanes past the row end are not
// counted. With K the number of leading bins holding at most cap entries,
// the candidates are the e >= kCandScale * 2^-K, all inside those bins since
// e <= kCandScale * 2^k for every k (K == kOctBins: every e > 0; K == 0: none).
constexpr float kCandScale = 1.41422f;  // > max of exp2q's polynomial over [-1/2, 1/2]

template <bool IN_ALL, int DT, int NVC>
__device__ __forceinline__ void exp_bins(const SampParams& p, ChunkSh& cs, float (&x)[NVC * Elem<DT>::kPerVec],
                                         int t, int nvc, float nmc) {
  constexpr int EPV = Elem<DT>::kPerVec;
  // byte offset of this lane's bin-0 word, the step per -bin and the
  // increment of its 16-bit half
  const int hi = t >> 5;
  const int hbase4 = ((t & 31) * kHistStride + (hi ? kOctBins - 1 : 0)) * 4;
  const int hstep4 = hi ? 4 : -4;
  const uint32_t hinc = hi ? 0x10000u : 1u;
  char* hist0 = reinterpret_cast<char*>(&cs.hist[0]);
#pragma unroll
  for (int u = 0; u < NVC; ++u) {
    const bool in = IN_ALL || u * kWave + t < nvc;
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      int ki;
      x[u * EPV + e] = exp2q_k(__builtin_fmaf(x[u * EPV + e], p.c, nmc), &ki);
      const int b = __builtin_elementwise_min(__builtin_elementwise_max(ki, -(kOctBins - 1)), 0);  // -bin
      if (in)
        __hip_atomic_fetch_add(reinterpret_cast<uint32_t*>(hist0 + (hbase4 + __mul24(hstep4, b))), hinc, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
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
}

// One chunk, processed by one wave: no workgroup barriers (the wave's LDS
// accesses are ordered; s_barrier of a one-wave workgroup only fences).
template <int DT, int NVC, bool PEN>
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
      if (PEN && ((pw[u] >> ((((u * kWave + t) * EPV) & 31) + e)) & 1u)) l = l < 0.0f ? l * p.pen : l * p.inv_pen;
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

  // 2. e in place, exponent bins, e-store
  if (full) {
    exp_bins<true, DT, NVC>(p, cs, x, t, nvc, nmc);
  } else {
    exp_bins<false, DT, NVC>(p, cs, x, t, nvc, nmc);
  }
  // chunk mass: each lane's 32 e pairwise, then the lanes pairwise
  const float mass = wave_tree_sum(lane_tree_sum(x));
  __syncthreads();

  // 3. bin totals: lane t < 32 (b = t & 15, q = t >> 4) sums word b of rows
  //    16q..16q+15 and clears it (both 16-bit halves at once: a half sums to
  //    at most 32 * 32); the low halves of word b count bin b of lanes 0..31,
  //    the high halves of word 15 - b bin b of lanes 32..63
  uint32_t bc;
  {
    const int b = t & (kOctBins - 1), q = (t >> 4) & 1;
    uint32_t sb = 0;
    if (t < kHistRows) {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        sb += __hip_atomic_exchange(&cs.hist[(16 * q + i) * kHistStride + b], 0u, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    sb += __shfl_xor(sb, 16);
    const uint32_t mirror = __shfl(sb, kOctBins - 1 - b);
    bc = t < kOctBins ? (sb & 0xffffu) + (mirror >> 16) : 0u;
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
  const float th = K >= kOctBins ? __uint_as_float(1u) : (K == 0 ? __builtin_inff() : __builtin_ldexpf(kCandScale, -K));
  // 5. candidate mask (bit 31 - i <-> element 32t + i), offsets
  uint32_t mask = 0;
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    // mask = 2 mask + (ec[i] >= th): a compare into VCC and one add with carry
    asm("v_cmp_ge_f32_e32 vcc, %1, %2\n\tv_addc_co_u32_e32 %0, vcc, %0, %0, vcc" : "+v"(mask) : "v"(ec[i]), "v"(th) : "vcc");
  }
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
template <int DT, bool PEN>
__global__ __launch_bounds__(kWave) __attribute__((amdgpu_waves_per_eu(kChunkWavesPerCu / 4)))
void chunk_kernel(const SampParams p) {
  constexpr int EPV = Elem<DT>::kPerVec;
  constexpr int NVC = kChunk / (kWave * EPV);  // vectors per lane: 8 (f32) or 4
  __shared__ ChunkSh cs;
  const int t = threadIdx.x;
  for (int i = t; i < kHistRows * kHistStride; i += kWave) cs.hist[i] = 0u;
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
    process_chunk<DT, NVC, PEN>(p, cs, item, cur, pcur, tcur);
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

// Shared memory of the row kernels: up to two rows (spec: the target and the
// draft row of one draft position) finalised side by side.
struct RowSh {
  uint64_t slot[2][kRowCand];          // candidate slots (idx << 32 | bits(p))
  union {
    uint64_t H[2][kBins];              // radix bins of each row
    float w[kRowCand];                 // draw weights per slot
  };
  float g[2][kMaxChunks];
  float mcj[2][kMaxChunks];
  uint32_t n[2][kMaxChunks];
  uint8_t kb[2][kMaxChunks];           // K of each chunk (kOctBins: complete)
  uint32_t gbits[2][kGather];
  uint64_t gw[2][kGather];
  uint32_t gcount[2];
  uint32_t sel32[2][2];
  uint64_t sel64[2][3];
  uint64_t red[2 * kRW];
  uint64_t red2[2 * kRW];              // block_sum_n's own buffer
  uint64_t red3[2 * kRW];              // the radix selects' own scan buffer
  uint64_t u64s[8];
  uint32_t u32s[8];
  float f32s[2][4];
  float slow_cut[2];
  float wmin[kRW];                     // per-wave minima (negated) of the slow path
  uint64_t slow_mass[2];
  uint64_t draws[64 + 1];
};

// Exclusive scans in lane order over the workgroup of NS values at once;
// tot receives the sums. smem holds NS * kRW words. LEAD = false drops the
// leading barrier, for a caller whose smem has a barrier between this and its
// previous use.
template <int NS, bool LEAD = true>
__device__ __forceinline__ void block_excl_scan_n(const uint64_t (&v)[NS], uint64_t* smem, uint64_t (&ex)[NS],
                                                  uint64_t (&tot)[NS]) {
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  uint64_t inc[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) inc[s] = wave_scan_add_u64(v[s]);
  if constexpr (LEAD) __syncthreads();
  if (lane == kWave - 1) {
#pragma unroll
    for (int s = 0; s < NS; ++s) smem[s * kRW + wid] = inc[s];
  }
  __syncthreads();
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    uint64_t base = 0, t = 0;
#pragma unroll
    for (int i = 0; i < kRW; ++i) {
      const uint64_t x = smem[s * kRW + i];
      base += i < wid ? x : 0;
      t += x;
    }
    ex[s] = base + inc[s] - v[s];
    tot[s] = t;
  }
}

// Sums over the workgroup of NS values at once, with one barrier. smem (NS *
// kRW words) must not be read by a wave still inside a previous use: the
// callers give it a buffer of its own.
template <int NS>
__device__ __forceinline__ void block_sum_n(const uint64_t (&v)[NS], uint64_t* smem, uint64_t (&tot)[NS]) {
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const uint64_t w = wave_scan_add_u64(v[s]);
    if (lane == kWave - 1) smem[s * kRW + wid] = w;
  }
  __syncthreads();
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    uint64_t t = 0;
#pragma unroll
    for (int i = 0; i < kRW; ++i) t += smem[s * kRW + i];
    tot[s] = t;
  }
}

__device__ __forceinline__ uint64_t block_excl_scan(uint64_t v, uint64_t* smem, uint64_t* total) {
  const uint64_t vv[1] = {v};
  uint64_t ex[1], tot[1];
  block_excl_scan_n<1>(vv, smem, ex, tot);
  *total = tot[0];
  return ex[0];
}

// Wave w: from the chunk records of row-set `set` (lane l holds records 2l
// and 2l+1) compute the row max, S and g_j (kept in sh.g / sh.mcj / sh.n),
// the bound on every p outside the candidates, and p of the draft token.
struct RowScale {
  float mcmax, s, p_bound, p_tok;
  bool has_tok;
};

__device__ __forceinline__ float chunk_bound(const ChunkRec& rec, float gj) {
  if (rec.flags & kChunkComplete) return 0.0f;
  return rec.K > 0 ? __builtin_ldexpf(kCandScale, -rec.K) * gj : __builtin_inff();
}

__device__ __forceinline__ RowScale row_scale(RowSh& sh, int set, const ChunkRec& ra, const ChunkRec& rb, int nch) {
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
    sh.g[set][ja] = ga;
    sh.mcj[set][ja] = ra.mc;
    sh.n[set][ja] = ra.n;
    sh.kb[set][ja] = static_cast<uint8_t>((ra.flags & kChunkComplete) ? kOctBins : ra.K);
  }
  if (ib) {
    sh.g[set][jb] = gb;
    sh.mcj[set][jb] = rb.mc;
    sh.n[set][jb] = rb.n;
    sh.kb[set][jb] = static_cast<uint8_t>((rb.flags & kChunkComplete) ? kOctBins : rb.K);
  }
  rs.p_bound = wave_max_f32(__builtin_fmaxf(ia ? chunk_bound(ra, ga) : 0.0f, ib ? chunk_bound(rb, gb) : 0.0f));
  const bool ta = ia && (ra.flags & kChunkHasTok), tb = ib && (rb.flags & kChunkHasTok);
  rs.has_tok = __ballot(ta || tb) != 0;
  rs.p_tok = wave_max_f32(ta ? ra.e_tok * ga : (tb ? rb.e_tok * gb : -1.0f));
  return rs;
}

// Chunk records 2l and 2l+1 of row r for lane l.
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

// Exact top-p cutoffs of NS sets at once (sets s0 .. s0+NS-1 of sh), each
// visited by visit(s, f), which passes f(bits, w) for its elements (bits of
// p > 0, w = fx46(p)): c = max{v : sum_{p >= v} w >= thr}, and the mass
// kept. Up to three radix rounds on the bits of p (12, 11 and 8 bits from the
// top; sh.H[s] zero on entry); after each round a bucket of at most kGather
// entries is finished by one wave (wave s for set s). found[s] is false when
// the set's total mass is below thr. The sets advance in lockstep, so NS rows
// cost the barriers of one. after_r0(d) runs on every lane once round 0 has
// found set 0's crossing digit d (the top 12 bits, bits >> kRound0Shift; kNone
// if the set holds less than thr): every element of p >= the cutoff has a
// digit >= d, so loads issued there for those elements overlap the rest.
constexpr int kRound0Shift = 19;

template <int NS, typename Visit, typename AfterR0>
__device__ void radix_select_n(RowSh& sh, int s0, const uint64_t (&thr)[NS], Visit visit, bool (&found)[NS],
                               float (&cut)[NS], uint64_t (&mass)[NS], AfterR0 after_r0) {
  const int t = threadIdx.x, lane = t & (kWave - 1), wid = t / kWave;
  uint32_t prefix[NS], pmask[NS];
  uint64_t above[NS];
  bool done[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    prefix[s] = pmask[s] = 0;
    above[s] = 0;
    done[s] = false;
    found[s] = false;
  }
  for (int round = 0; round < 3; ++round) {
    const int shift = round == 0 ? kRound0Shift : (round == 1 ? 8 : 0);
    const uint32_t dmask = round == 0 ? 0xfffu : (round == 1 ? 0x7ffu : 0xffu);
    if (round > 0) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        if (!done[s]) {
#pragma unroll
          for (int q = 0; q < kBinsPerLane; ++q) sh.H[s0 + s][kBinsPerLane * t + q] = 0;
        }
      }
      __syncthreads();
    }
    // this round's crossing digit and gather count start empty (the barrier
    // below orders these stores before any use)
    if (t < NS) {
      sh.sel32[t][0] = kNone;
      sh.gcount[t] = 0;
    }
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (!done[s]) {
        uint64_t* H = sh.H[s0 + s];
        const uint32_t pm = pmask[s], pf = prefix[s];
        visit(s, [&](uint32_t bits, uint64_t w) {
          if ((bits & pm) == pf && w)
            __hip_atomic_fetch_add(&H[digit_of(bits, shift, dmask)], w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        });
      }
    }
    __syncthreads();
    // lane t owns digits kBins-1 - (kBinsPerLane*t + q), q = 0.. (descending)
    uint64_t v[NS][kBinsPerLane], sum[NS], ex[NS], tot[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      sum[s] = 0;
#pragma unroll
      for (int q = 0; q < kBinsPerLane; ++q) {
        v[s][q] = done[s] ? 0 : sh.H[s0 + s][kBins - 1 - (kBinsPerLane * t + q)];
        sum[s] += v[s][q];
      }
    }
    block_excl_scan_n<NS, false>(sum, sh.red3, ex, tot);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      uint64_t before = above[s] + ex[s];
      if (!done[s] && before < thr[s] && before + sum[s] >= thr[s]) {
#pragma unroll
        for (int q = 0; q < kBinsPerLane; ++q) {
          if (before < thr[s] && before + v[s][q] >= thr[s]) {
            sh.sel32[s][0] = static_cast<uint32_t>(kBins - 1 - (kBinsPerLane * t + q));
            sh.sel64[s][0] = before;
            sh.sel64[s][1] = v[s][q];
          }
          before += v[s][q];
        }
      }
    }
    __syncthreads();
    uint64_t binmass[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      binmass[s] = 0;
      if (!done[s]) {
        const uint32_t digit = sh.sel32[s][0];
        if (digit == kNone) {
          done[s] = true;
        } else {
          prefix[s] |= digit << shift;
          pmask[s] |= dmask << shift;
          above[s] = sh.sel64[s][0];
          binmass[s] = sh.sel64[s][1];
        }
      }
    }
    if (round == 0) after_r0(sh.sel32[0][0]);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (!done[s]) {
        const uint32_t pm = pmask[s], pf = prefix[s];
        uint32_t* gb = sh.gbits[s];
        uint64_t* gw = sh.gw[s];
        uint32_t* gc = &sh.gcount[s];
        visit(s, [&](uint32_t bits, uint64_t w) {
          if ((bits & pm) == pf && w) {
            const uint32_t k = __hip_atomic_fetch_add(gc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            if (k < kGather) {
              gb[k] = bits;
              gw[k] = w;
            }
          }
        });
      }
    }
    __syncthreads();
    bool finish[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      finish[s] = false;
      if (!done[s]) {
        const uint32_t cnt = sh.gcount[s];
        if (cnt > kGather && round == 2) {
          // every entry of the bucket has the same bits
          cut[s] = __uint_as_float(prefix[s]);
          mass[s] = above[s] + binmass[s];
          found[s] = true;
          done[s] = true;
        } else if (cnt <= kGather) {
          finish[s] = true;
          if (wid == s) {
            const uint32_t b = lane < static_cast<int>(cnt) ? sh.gbits[s][lane] : 0u;
            uint64_t A = above[s];
            for (int j = 0; j < static_cast<int>(cnt); ++j) {
              const uint32_t bj = sh.gbits[s][j];
              const uint64_t wj = sh.gw[s][j];
              A += bj >= b ? wj : 0;
            }
            const bool ok = lane < static_cast<int>(cnt) && A >= thr[s];
            const uint64_t best = wave_max_u64(ok ? b : 0u);
            const uint64_t at = wave_max_u64(ok && b == static_cast<uint32_t>(best) ? A : 0);
            if (lane == 0) {
              sh.sel32[s][1] = static_cast<uint32_t>(best);
              sh.sel64[s][2] = at;
            }
          }
        }
      }
    }
    __syncthreads();
    bool all = true;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (finish[s]) {
        cut[s] = __uint_as_float(sh.sel32[s][1]);
        mass[s] = sh.sel64[s][2];
        found[s] = true;
        done[s] = true;
      }
      all = all && done[s];
    }
    if (all) break;
  }
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

// Index-ordered inverse-CDF pick over the first n slots; weight(s) is an
// exact fx46 mass. Lane t owns slots [8t, 8t+8). Returns the winning slot, or
// -1 at zero total mass.
template <typename W>
__device__ int pick_slot(RowSh& sh, int n, float u, W weight) {
  const int t = threadIdx.x;
  const int s0 = kSlotsPerLane * t;
  uint64_t sum = 0;
#pragma unroll
  for (int q = 0; q < kSlotsPerLane; ++q) sum += s0 + q < n ? weight(s0 + q) : 0;
  // the scan's barrier publishes this before any lane can set it
  if (t == 0) sh.u32s[3] = kNone;
  const uint64_t vv[1] = {sum};
  uint64_t exv[1], totv[1];
  // no leading barrier: every caller reaches this through a barrier after
  // its last other use of sh.red
  block_excl_scan_n<1, false>(vv, sh.red, exv, totv);
  const uint64_t ex = exv[0], total = totv[0];
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
__device__ int64_t pick_dense(RowSh& sh, int vocab, float u, W weight) {
  const int t = threadIdx.x;
  const int per = (vocab + kRB - 1) / kRB;
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

// The candidates' cutoff cut of the row of set `set` did not clear the
// worst-case bound on the p outside the candidates. Re-reads only the chunks
// whose bound reaches cut and checks their non-candidates exactly: true iff
// every p outside the candidates is below cut, in which case cut and the
// candidates' mass are the row's (no element outside the candidates can
// reach a value >= cut). Runs inside slow_select.
template <int DT>
__device__ __forceinline__ bool bound_repair(RowSh& sh, int set, const char* rowp, const uint32_t* bm, float c,
                                             float pen, float inv_pen, int vocab, int nch, float cut) {
  const int t = threadIdx.x;
  bool bad = false;
  for (int j = 0; j < nch; ++j) {
    const int K = sh.kb[set][j];
    if (K >= kOctBins) continue;
    const float gj = sh.g[set][j];
    const float th = K > 0 ? __builtin_ldexpf(kCandScale, -K) : __builtin_inff();
    if (K > 0 && !(th * gj >= cut)) continue;  // chunk_bound below cut
    const float nmc = -sh.mcj[set][j];
    const int c0 = j * kChunk;
#pragma unroll
    for (int q = 0; q < kChunk / kRB; ++q) {
      const int i = c0 + t + q * kRB;
      if (i < vocab) {
        float l = load_elem<DT>(rowp, i);
        if (bm && bit_of(bm, i)) l = l < 0.0f ? l * pen : l * inv_pen;
        const float e = exp2q(__builtin_fmaf(l, c, nmc));
        bad = bad || (!(e >= th) && e * gj >= cut);
      }
    }
  }
  // block-wide OR through LDS (no device-library call)
  if (t == 0) sh.u32s[6] = 0u;
  __syncthreads();
  if (bad) sh.u32s[6] = 1u;
  __syncthreads();
  const bool any = sh.u32s[6] != 0u;
  __syncthreads();
  return !any;
}

// Chunk rebuild, when the bound repair found a non-candidate p >= cut (the
// candidates' cutoff): the candidates of every chunk whose bound reaches cut
// become {p >= cut} of that chunk, in index order, if they fit its cap slots.
// cut is a lower bound of the row's cutoff (the candidates alone hold top_p
// at p >= cut), and the other chunks hold no p >= cut, so afterwards the
// slots hold every element of p >= the row's cutoff and their select is exact.
// Returns false (slots partly rewritten) if some chunk does not fit. Out of
// line, like slow_select.
template <int DT, int OCC>
__device__ __noinline__ bool rebuild_chunks(RowSh& sh, int set, const char* rowp, const uint32_t* bm, float c,
                                               float pen, float inv_pen, int vocab, int nch, int cap, float cut) {
  constexpr int kQ = kChunk / kRB;
  static_assert(kQ * kRW <= kGather, "per-(q, wave) counts fit sh.gbits[0]");
  const int t = threadIdx.x, lane = t & (kWave - 1), wid = t / kWave;
  // at fixed offsets (sets are rebuilt one at a time), so the count reads
  // take immediate offsets rather than per-read addresses
  uint32_t* cnt = sh.gbits[0];
#pragma nounroll
  for (int j = 0; j < nch; ++j) {
    const int K = sh.kb[set][j];
    if (K >= kOctBins) continue;
    const float gj = sh.g[set][j];
    const float th = K > 0 ? __builtin_ldexpf(kCandScale, -K) : __builtin_inff();
    if (K > 0 && !(th * gj >= cut)) continue;  // chunk_bound below cut
    const float nmc = -sh.mcj[set][j];
    const int c0 = j * kChunk;
    float pq[kQ];
    uint64_t mq[kQ];
#pragma unroll
    for (int q = 0; q < kQ; ++q) {
      // element c0 + q*kRB + t: (q, t) order is index order
      const int i = c0 + t + q * kRB;
      pq[q] = 0.0f;
      if (i < vocab) {
        float l = load_elem<DT>(rowp, i);
        if (bm && bit_of(bm, i)) l = l < 0.0f ? l * pen : l * inv_pen;
        pq[q] = exp2q(__builtin_fmaf(l, c, nmc)) * gj;
      }
      mq[q] = __ballot(pq[q] > 0.0f && pq[q] >= cut);
      if (lane == 0) cnt[q * kRW + wid] = static_cast<uint32_t>(__builtin_popcountll(mq[q]));
    }
    __syncthreads();
    // lane l < kQ*kRW holds count l = (q, w) in (q, t) order; an inclusive
    // scan over the lanes gives each wave base[q], the flagged elements
    // before its own of round q
    int incl = lane < kQ * kRW ? static_cast<int>(cnt[lane]) : 0;
#pragma unroll
    for (int d = 1; d < kQ * kRW; d <<= 1) {
      const int o = __shfl_up(incl, d);
      incl += lane >= d ? o : 0;
    }
    const int total = __shfl(incl, kQ * kRW - 1);
    int base[kQ];
#pragma unroll
    for (int q = 0; q < kQ; ++q) {
      const int l = q * kRW + wid;
      base[q] = __shfl(incl, l) - static_cast<int>(cnt[l]);
    }
    if (total > cap) {
      __syncthreads();  // every wave is past its reads of cnt
      return false;
    }
    uint64_t* slots = sh.slot[set] + j * cap;
#pragma unroll
    for (int q = 0; q < kQ; ++q) {
      if ((mq[q] >> lane) & 1u) {
        const int pos = base[q] + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                                      static_cast<uint32_t>(mq[q] >> 32),
                                      __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mq[q]), 0u)));
        slots[pos] = (static_cast<uint64_t>(c0 + t + q * kRB) << 32) | __float_as_uint(pq[q]);
      }
    }
    if (t >= total && t < cap) slots[t] = 0;
    if (t == 0) {
      sh.n[set][j] = static_cast<uint32_t>(total);
      sh.kb[set][j] = static_cast<uint8_t>(kOctBins);
    }
    __syncthreads();  // slots written; cnt free for the next chunk
  }
  return true;
}

// Cutoff of the row of set `set` when its candidates' cutoff did not pass the
// bound. mode kSlowCand: the candidates' select again; if they hold top_p,
// the bound repair returns kRepaired when their cutoff stands, else
// kNeedRebuild (for the chunk rebuild, then mode kSlowRebuilt: the select over
// the rebuilt slots, exact, returns kRebuilt). Otherwise (and in mode
// kSlowRow) the exact select over every element of the row, p recomputed from
// the re-read logits with the set's g_j; when keep is set, it leaves the
// support {p >= c} in index order in sh.slot[set] (as idx << 32 | bits(p))
// and returns its size, or -1 if it does not fit. The cutoff and its fx46
// mass go to sh.slow_cut / sh.slow_mass. Out of line, with plain arguments
// and no pointers into the caller's frame, so the common path's registers are
// unaffected.
constexpr int kRepaired = -2;     // the candidates' cutoff stands
constexpr int kRebuilt = -3;      // the rebuilt slots' cutoff
constexpr int kNeedRebuild = -4;  // the candidates hold top_p but a non-candidate reaches their cutoff
enum SlowMode : int { kSlowCand = 0, kSlowRebuilt = 1, kSlowRow = 2 };

template <int DT, int OCC>
__device__ __noinline__ int slow_select(RowSh& sh, int set, const char* rowp, const uint32_t* bm, float c, float pen,
                                        float inv_pen, int vocab, int nch, int nslots, uint64_t thr, bool keep,
                                        int mode) {
  const int t = threadIdx.x, wid = t / kWave;
  const float* mcj = sh.mcj[set];
  const float* gj = sh.g[set];
  auto pval = [&](int i) { return p_elem<DT>(rowp, bm, c, pen, inv_pen, mcj, gj, i); };
  const uint64_t thr1[1] = {thr};
  bool found[1];
  float cc1[1];
  uint64_t mfx1[1];
  // 1. the select over the slots (the candidates' p are still in
  //    sh.slot[set], or the rebuilt chunks')
  if (mode != kSlowRow) {
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kBinsPerLane; ++q) sh.H[set][kBinsPerLane * t + q] = 0;
    __syncthreads();
    radix_select_n<1>(sh, set, thr1, [&](int, auto f) {
      for (int sl = t; sl < nslots; sl += kRB) {
        const uint32_t bits = static_cast<uint32_t>(sh.slot[set][sl]);
        const float x = __uint_as_float(bits);
        if (x > 0.0f) f(bits, fx46(x));
      }
    }, found, cc1, mfx1, [](uint32_t) {});
    if (found[0]) {
      if (mode == kSlowCand && !bound_repair<DT>(sh, set, rowp, bm, c, pen, inv_pen, vocab, nch, cc1[0])) {
        if (t == 0) sh.slow_cut[set] = cc1[0];
        __syncthreads();
        return kNeedRebuild;
      }
      if (t == 0) {
        sh.slow_cut[set] = cc1[0];
        sh.slow_mass[set] = mfx1[0];
      }
      __syncthreads();
      return mode == kSlowCand ? kRepaired : kRebuilt;
    }
  }
  // 2. exact select over the whole row
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kBinsPerLane; ++q) sh.H[set][kBinsPerLane * t + q] = 0;
  __syncthreads();
  radix_select_n<1>(sh, set, thr1, [&](int, auto f) {
    for (int i = t; i < vocab; i += kRB) {
      const float pv = pval(i);
      f(__float_as_uint(pv), fx46(pv));
    }
  }, found, cc1, mfx1, [](uint32_t) {});
  float cc = cc1[0];
  uint64_t mfx = mfx1[0];
  if (!found[0]) {
    // Total mass below the threshold: keep the whole row (cutoff = min p).
    float mn = __builtin_inff();
    uint64_t tot = 0;
    for (int i = t; i < vocab; i += kRB) {
      const float pv = pval(i);
      mn = fminf(mn, pv);
      tot += fx46(pv);
    }
    mn = wave_max_f32(-mn);
    if ((t & (kWave - 1)) == 0) sh.wmin[wid] = mn;
    uint64_t all;
    (void)block_excl_scan(tot, sh.red, &all);  // its barriers also publish wmin
    float m = sh.wmin[0];
#pragma unroll
    for (int w = 1; w < kRW; ++w) m = nmax(m, sh.wmin[w]);
    cc = -m;
    mfx = all;
    __syncthreads();
  }
  if (t == 0) {
    sh.slow_cut[set] = cc;
    sh.slow_mass[set] = mfx;
  }
  __syncthreads();
  if (!keep) return -1;
  const int per = (vocab + kRB - 1) / kRB;
  const int a = t * per < vocab ? t * per : vocab;
  const int b = a + per < vocab ? a + per : vocab;
  uint64_t cnt = 0;
  for (int i = a; i < b; ++i) cnt += pval(i) >= cc ? 1 : 0;
  uint64_t total;
  const uint64_t ex = block_excl_scan(cnt, sh.red, &total);
  if (total > static_cast<uint64_t>(kRowCand)) {
    __syncthreads();  // every wave is past its reads of sh.red
    return -1;
  }
  int pos = static_cast<int>(ex);
  for (int i = a; i < b; ++i) {
    const float pv = pval(i);
    if (pv >= cc) sh.slot[set][pos++] = (static_cast<uint64_t>(i) << 32) | __float_as_uint(pv);
  }
  __syncthreads();
  return static_cast<int>(total);
}

// Candidate slot s of row r: (idx << 32 | bits(e)); stale beyond n_j.
__device__ __forceinline__ uint64_t load_slot(const SampParams& p, int64_t r, int s) {
  return p.cands[(r * p.nch + (s >> p.cap_log2)) * kChunkCand + (s & (p.cap - 1))];
}

__device__ __forceinline__ bool slot_valid(const RowSh& sh, int set, const SampParams& p, int s) {
  return (s & (p.cap - 1)) < static_cast<int>(sh.n[set][s >> p.cap_log2]);
}

// Finalisation of NS rows side by side (set s = row r[s]): scales, p of the
// candidates into sh.slot[s] (idx << 32 | bits(p), 0 for empty slots), the
// exact top-p cutoff (candidates, or the re-streamed row when they do not hold
// it). after_r0 is the candidates' select's round-0 hook (set 0's crossing
// digit). Outputs the row statistics, the filtered probability of each row's
// draft token (-1 if the row has none) and, for a row that took the slow path
// with keep_support, the size of its support.
template <int DT, int NS, int OCC, typename AfterR0>
__device__ void finalize_rows(const SampParams& p, RowSh& sh, const int64_t (&r)[NS], bool keep_support,
                              RowStat (&st)[NS], float (&P_tok)[NS], int (&n_sup)[NS], AfterR0 after_r0) {
  const int t = threadIdx.x, wid = t / kWave;
  const int nch = p.nch;
  const int nslots = nch * p.cap;
  float top_p[NS];
  bool unf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    top_p[s] = p.top_p_rows ? p.top_p_rows[r[s]] : p.top_p;
    unf[s] = !(top_p[s] < 1.0f);
  }
  // 1. chunk records (wave s: row s) and candidate slots (strided), in flight together
  ChunkRec ra{}, rb{};
  if (wid < NS) load_recs(p, wid == 0 ? r[0] : r[NS - 1], &ra, &rb);
  uint64_t cv[NS][kSlotsPerLane];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
#pragma unroll
    for (int q = 0; q < kSlotsPerLane; ++q) {
      const int sl = t + q * kRB;
      cv[s][q] = (!unf[s] && sl < nslots) ? load_slot(p, r[s], sl) : 0;
    }
#pragma unroll
    for (int q = 0; q < kBinsPerLane; ++q) sh.H[s][kBinsPerLane * t + q] = 0;
  }
  // 2. row scales (wave s: row s)
  if (wid < NS) {
    const RowScale rs = row_scale(sh, wid, ra, rb, nch);
    if ((t & (kWave - 1)) == 0) {
      sh.f32s[wid][0] = rs.mcmax;
      sh.f32s[wid][1] = rs.s;
      sh.f32s[wid][2] = rs.p_bound;
      sh.f32s[wid][3] = rs.has_tok ? rs.p_tok : -1.0f;
    }
  }
  __syncthreads();
  // 3. p of the candidates, kept in registers and in sh.slot
  float pv[NS][kSlotsPerLane];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
#pragma unroll
    for (int q = 0; q < kSlotsPerLane; ++q) {
      const int sl = t + q * kRB;
      pv[s][q] = 0.0f;
      if (!unf[s] && sl < nslots && slot_valid(sh, s, p, sl))
        pv[s][q] = __uint_as_float(static_cast<uint32_t>(cv[s][q])) * sh.g[s][sl >> p.cap_log2];
      if (sl < nslots) sh.slot[s][sl] = ((cv[s][q] >> 32) << 32) | __float_as_uint(pv[s][q]);
    }
  }
  // 4. cutoffs
  uint64_t thr[NS];
  bool found[NS];
  float cut[NS];
  uint64_t mfx[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) thr[s] = unf[s] ? 0 : fx46(top_p[s]);
  bool any = false;
#pragma unroll
  for (int s = 0; s < NS; ++s) any = any || !unf[s];
  if (any) {
    radix_select_n<NS>(sh, 0, thr, [&](int s, auto f) {
#pragma unroll
      for (int q = 0; q < kSlotsPerLane; ++q) {
        const float x = pv[s][q];
        if (x > 0.0f) f(__float_as_uint(x), fx46(x));
      }
    }, found, cut, mfx, after_r0);
  }
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    st[s].mcmax = sh.f32s[s][0];
    st[s].s = sh.f32s[s][1];
    st[s].flags = unf[s] ? (kFlagUnfiltered | kFlagDense) : 0u;
    st[s].cutoff = 0.0f;
    st[s].mass_fx = 0;
    n_sup[s] = nslots;
    const float p_bound = sh.f32s[s][2];
    if (!unf[s]) {
      if (found[s] && cut[s] > p_bound) {
        st[s].cutoff = cut[s];
        st[s].mass_fx = mfx[s];
      } else {
        const int64_t g = r[s] / p.rpg;
        const uint32_t* bm = p.use_pen ? p.bitmap + g * p.bm_words : nullptr;
        const char* rowp = row_of(p, g, static_cast<int>(r[s] - g * p.rpg));
        int n = slow_select<DT, OCC>(sh, s, rowp, bm, p.c, p.pen, p.inv_pen, p.vocab, nch, nslots, thr[s], keep_support,
                                kSlowCand);
        if (n == kNeedRebuild) {
          // the deficient chunks' candidates become {p >= the candidates' cutoff}
          const bool fits = rebuild_chunks<DT, OCC>(sh, s, rowp, bm, p.c, p.pen, p.inv_pen, p.vocab, nch, p.cap,
                                               sh.slow_cut[s]);
          n = slow_select<DT, OCC>(sh, s, rowp, bm, p.c, p.pen, p.inv_pen, p.vocab, nch, nslots, thr[s], keep_support,
                              fits ? kSlowRebuilt : kSlowRow);
        }
        st[s].cutoff = sh.slow_cut[s];
        st[s].mass_fx = sh.slow_mass[s];
        const bool rep = n == kRepaired, reb = n == kRebuilt;
        st[s].flags |= rep ? 0u : (reb ? kFlagRebuilt : (kFlagSlow | ((!keep_support || n < 0) ? kFlagDense : 0u)));
        n_sup[s] = rep || reb ? nslots : n;
      }
    }
    st[s].mass = unf[s] ? 1.0f : mass_to_f32(st[s].mass_fx);
    const float pt = sh.f32s[s][3];
    P_tok[s] = pt < 0.0f ? -1.0f : (unf[s] ? pt : (pt >= st[s].cutoff ? pt / st[s].mass : 0.0f));
    st[s].p_tok = P_tok[s] < 0.0f ? 0.0f : P_tok[s];
  }
}

// Inverse-CDF draw over the row of set `set` (its slots hold idx | bits(p),
// n of them, sh.g / sh.mcj its scales): weights fx46(P), P the filtered,
// renormalised probability; the whole row when it is dense.
template <int DT>
__device__ int64_t own_draw(const SampParams& p, RowSh& sh, int set, const RowStat& st, int n, float u,
                            const char* rowp, const uint32_t* bm) {
  const bool unf = st.flags & kFlagUnfiltered;
  const float cc = st.cutoff, mass = st.mass;
  if (!(st.flags & kFlagDense)) {
    const int win = pick_slot(sh, n, u, [&](int s) {
      const float x = __uint_as_float(static_cast<uint32_t>(sh.slot[set][s]));
      return x >= cc && x > 0.0f ? fx46(x / mass) : 0ull;
    });
    return win < 0 ? 0 : static_cast<int64_t>(sh.slot[set][win] >> 32);
  }
  return pick_dense(sh, p.vocab, u, [&](int i) {
    const float x = p_elem<DT>(rowp, bm, p.c, p.pen, p.inv_pen, sh.mcj[set], sh.g[set], i);
    return fx46(unf ? x : (x >= cc ? x / mass : 0.0f));
  });
}

// Publish draw word w of group g and arrive on its counter; the last of the
// k+1 arrivals runs the accept chain: a = the first position whose accept
// bit (bit 63) is clear, tokens = the accepted drafts, draw a, then -1.
__device__ void publish_draw(const SampParams& p, RowSh& sh, int64_t g, int i, uint64_t word) {
  const int k = p.k;
  const int t = threadIdx.x, lane = t & (kWave - 1), wid = t / kWave;
  if (t == 0) {
    store_sc64(reinterpret_cast<uint64_t*>(p.draws) + g * (k + 1) + i, word);
    drain_stores();
    uint32_t* ctr = p.grp_cnt + g * kCounterStride;
    const uint32_t prev = atomic_arrive(ctr);
    const bool last = prev == static_cast<uint32_t>(k);
    if (last) store_sc(ctr, 0u);
    sh.u32s[7] = last ? 1u : 0u;
  }
  __syncthreads();
  if (!sh.u32s[7] || wid != 0) return;
  // wave 0 alone: lane l holds draw l (lane 0 also draw 64 when k == 64)
  const uint64_t* dw = reinterpret_cast<const uint64_t*>(p.draws) + g * (k + 1);
  const uint64_t d = lane <= k ? load_sc64(dw + lane) : 0;
  const uint64_t d64 = (k >= kWave && lane == 0) ? load_sc64(dw + kWave) : 0;
  const int64_t x = lane < k ? p.draft_tokens[g * k + lane] : -1;
  const uint64_t bad = __ballot(lane < k && !(d >> 63));
  const int a = bad ? __builtin_ctzll(bad) : k;
  const uint64_t wa = a < kWave ? __shfl(d, a) : __shfl(d64, 0);
  const int64_t da = static_cast<int64_t>(wa & ~(1ull << 63));
  int64_t* out = p.tokens + g * (k + 1);
  if (lane < a) out[lane] = x;
  if (lane == a) out[lane] = da;
  if (lane > a && lane <= k) out[lane] = -1;
  if (k >= kWave && lane == 0) out[k] = a == k ? da : -1;
  if (lane == 0) p.accept_len[g] = a;
}

// Spec mode: one workgroup per (batch element g, position i). i < k: the
// target row i and the draft row i, finalised side by side; the accept bit
// of draft token x_i (u < min(1, P/Q), sampler.py:451-452) and the residual
// draw normalize(max(P - Q, 0)) (fallback normalize(P), rejection.py:60-69)
// with u[g, k+i]. i == k: the bonus row's draw with u[g, 2k].
// OCC = 4: built for two workgroups per CU (at most 128 registers, the
// out-of-line slow path in its own copies), launched when the workgroups
// outnumber the CUs; OCC = 0 otherwise (no spills).
template <int DT, int OCC>
__global__ __launch_bounds__(kRB) __attribute__((amdgpu_waves_per_eu(OCC > 0 ? OCC : 1)))
void spec_row_kernel(const SampParams p) {
  __shared__ RowSh sh;
  const int k = p.k, rpg = 2 * k + 1;
  const int64_t g = blockIdx.x / (k + 1);
  const int i = static_cast<int>(blockIdx.x - g * (k + 1));
  const int t = threadIdx.x;
  const int nslots = p.nch * p.cap;
  const uint32_t* bm = p.use_pen ? p.bitmap + g * p.bm_words : nullptr;
  // this workgroup's scalars, loaded before the row work so that their latency
  // is not paid after it
  const float u_acc = p.uniforms[g * rpg + i];        // i < k: acceptance draw
  const float u_draw = p.uniforms[g * rpg + k + i];   // residual draw (bonus draw u[2k] when i == k)
  const int64_t x = i < k ? p.draft_tokens[g * k + i] : -1;
  const bool bonus = i == k;
  const int64_t r[2] = {g * rpg + (bonus ? k : i), g * rpg + (bonus ? k : k + 1 + i)};
  const char* trow = row_of(p, g, bonus ? k : i);
  const char* drow = row_of(p, g, bonus ? k : k + 1 + i);
  // the draft logits' bits at the target's candidates that can be in its
  // support (digit >= the target select's round-0 crossing digit d0), gathered
  // during the rest of the select and decoded at their use (the bonus
  // workgroup has no draft row)
  uint32_t lq[kSlotsPerLane] = {};
  auto gather = [&](uint32_t d0) {
    if (bonus || d0 == kNone) return;
#pragma unroll
    for (int q = 0; q < kSlotsPerLane; ++q) {
      const int sl = t + q * kRB;
      if (sl < nslots) {
        const uint64_t v = sh.slot[0][sl];
        const uint32_t bits = static_cast<uint32_t>(v);
        if (bits != 0u && (bits >> kRound0Shift) >= d0) {
          const int idx = static_cast<int>(v >> 32);
          lq[q] = load_bits<DT>(drow, idx < p.vocab ? idx : 0);
        }
      }
    }
  };
  RowStat st[2];
  float P_tok[2];
  int n_sup[2];
  // keep_support: a row whose cutoff needed the whole-row select keeps its
  // support (if it fits the slots) in index order, so its draw stays on slots
  finalize_rows<DT, 2, OCC>(p, sh, r, true, st, P_tok, n_sup, gather);
  // target slots: the candidates, or the kept support of a slow row
  const int nt = (st[0].flags & kFlagSlow) ? n_sup[0] : nslots;
  if (bonus) {
    const int64_t tok = own_draw<DT>(p, sh, 0, st[0], nt, u_draw, trow, bm);
    publish_draw(p, sh, g, k, static_cast<uint64_t>(tok));
    return;
  }
  if ((st[0].flags & kFlagRebuilt) || (st[0].flags & (kFlagSlow | kFlagDense)) == kFlagSlow) {
    // the support or rebuilt chunks replaced candidates: gather the draft
    // logits again (slots with p > 0 hold token indices)
#pragma unroll
    for (int q = 0; q < kSlotsPerLane; ++q) {
      const int sl = t + q * kRB;
      lq[q] = 0u;
      if (sl < nt) {
        const uint64_t v = sh.slot[0][sl];
        if (static_cast<uint32_t>(v) != 0u) {
          const int idx = static_cast<int>(v >> 32);
          lq[q] = load_bits<DT>(drow, idx < p.vocab ? idx : 0);
        }
      }
    }
  }
  const RowStat& st_t = st[0];
  const RowStat& st_d = st[1];
  // accept bit of x_i
  const bool acc = x >= 0 && x < p.vocab && accept_draw(u_acc, P_tok[0] < 0.0f ? 0.0f : P_tok[0],
                                                        P_tok[1] < 0.0f ? 0.0f : P_tok[1]);
  const float u = u_draw;
  const bool unf_t = st_t.flags & kFlagUnfiltered;
  const bool unf_d = st_d.flags & kFlagUnfiltered;
  auto Qof = [&](float l, int idx) {
    if (bm && bit_of(bm, idx)) l = l < 0.0f ? l * p.pen : l * p.inv_pen;
    const int j = idx >> kChunkShift;
    const float q = exp2q(__builtin_fmaf(l, p.c, -sh.mcj[1][j])) * sh.g[1][j];
    return unf_d ? q : (q >= st_d.cutoff ? q / st_d.mass : 0.0f);
  };
  int64_t token;
  if (!(st_t.flags & kFlagDense)) {
    float P[kSlotsPerLane], D[kSlotsPerLane];
    uint64_t sums[2] = {0, 0};  // fx46 masses of D and of P
#pragma unroll
    for (int q = 0; q < kSlotsPerLane; ++q) {
      const int sl = t + q * kRB;
      P[q] = D[q] = 0.0f;
      if (sl < nt) {
        const uint64_t v = sh.slot[0][sl];
        const float pv = __uint_as_float(static_cast<uint32_t>(v));
        if (pv > 0.0f && pv >= st_t.cutoff) {
          P[q] = pv / st_t.mass;
          const float dv = P[q] - Qof(bits_to_float<DT>(lq[q]), static_cast<int>(v >> 32));
          D[q] = dv > 0.0f ? dv : 0.0f;
          sums[0] += fx46(D[q]);
          sums[1] += fx46(P[q]);
        }
      }
    }
    uint64_t tot[2];
    block_sum_n<2>(sums, sh.red2, tot);
    const bool use_d = tot[0] > 0;
    const float den = use_d ? mass_to_f32(tot[0]) : (tot[1] > 0 ? mass_to_f32(tot[1]) : 1.0f);
#pragma unroll
    for (int q = 0; q < kSlotsPerLane; ++q) {
      // both values in registers first: a select of the two arrays would
      // otherwise become a select of their addresses, on the stack
      float dq = D[q], pq = P[q];
      asm volatile("" : "+v"(dq), "+v"(pq));
      const int sl = t + q * kRB;
      if (sl < nt) sh.w[sl] = (use_d ? dq : pq) / den;
    }
    __syncthreads();
    const int win = pick_slot(sh, nt, u, [&](int s) { return fx46(sh.w[s]); });
    token = win < 0 ? 0 : static_cast<int64_t>(sh.slot[0][win] >> 32);
  } else {
    // dense target row: the whole vocabulary
    auto Pof = [&](int y) {
      const float pv = p_elem<DT>(trow, bm, p.c, p.pen, p.inv_pen, sh.mcj[0], sh.g[0], y);
      return unf_t ? pv : (pv >= st_t.cutoff ? pv / st_t.mass : 0.0f);
    };
    auto Qat = [&](int y) { return Qof(load_elem<DT>(drow, y), y); };
    uint64_t sums[2] = {0, 0};
    {
      const int per = (p.vocab + kRB - 1) / kRB;
      const int i0 = t * per < p.vocab ? t * per : p.vocab;
      const int i1 = i0 + per < p.vocab ? i0 + per : p.vocab;
      for (int y = i0; y < i1; ++y) {
        const float pj = Pof(y);
        const float dj = pj - Qat(y);
        sums[0] += fx46(dj > 0.0f ? dj : 0.0f);
        sums[1] += fx46(pj);
      }
    }
    uint64_t ex[2], tot[2];
    block_excl_scan_n<2>(sums, sh.red, ex, tot);
    const bool use_d = tot[0] > 0;
    const float den = use_d ? mass_to_f32(tot[0]) : (tot[1] > 0 ? mass_to_f32(tot[1]) : 1.0f);
    token = pick_dense(sh, p.vocab, u, [&](int y) {
      const float pj = Pof(y);
      float v = pj;
      if (use_d) {
        const float dj = pj - Qat(y);
        v = dj > 0.0f ? dj : 0.0f;
      }
      return fx46(v / den);
    });
  }
  publish_draw(p, sh, g, i, static_cast<uint64_t>(token) | (acc ? 1ull << 63 : 0ull));
}

// Sample and dense modes: one workgroup per row.
template <int DT, int MODE>
__global__ __launch_bounds__(kRB) void row_kernel(const SampParams p) {
  __shared__ RowSh sh;
  const int64_t r[1] = {blockIdx.x};
  const int t = threadIdx.x;
  RowStat st[1];
  float P_tok[1];
  int n_sup[1];
  finalize_rows<DT, 1, 0>(p, sh, r, MODE == kModeSample, st, P_tok, n_sup, [](uint32_t) {});
  if constexpr (MODE == kModeSample) {
    const uint32_t* bm = p.use_pen ? p.bitmap + r[0] * p.bm_words : nullptr;
    const int64_t token = own_draw<DT>(p, sh, 0, st[0], (st[0].flags & kFlagSlow) ? n_sup[0] : p.nch * p.cap,
                                       p.row_uniforms[r[0]], row_of(p, r[0], 0), bm);
    if (t == 0) p.row_tokens[r[0]] = token;
  } else {
    if (t == 0) {
      p.stats[r[0]] = st[0];
      const bool unf = st[0].flags & kFlagUnfiltered;
      if (p.cutoff_out) p.cutoff_out[r[0]] = unf ? 0.0f : st[0].cutoff;
      if (p.mass_out) p.mass_out[r[0]] = st[0].mass;
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
  uint64_t grp_cnt, chunks, cands, stats, draws, bitmap, total;
};

// Workspace: [group arrival counters, one 64-byte line each, for up to
// kMaxSpecBatch batch elements] (at a fixed place, so calls of any shape find
// them zero) [chunk records] [candidates] [row statistics] [draws] [penalty
// bitmaps, one per group].
Layout ws_layout(int64_t rows, int64_t groups, int nch) {
  auto al = [](uint64_t x) { return (x + 255u) & ~255ull; };
  Layout l{};
  l.grp_cnt = 0;
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
  const dim3 grid(p.items < wgs ? p.items : wgs);
  if (p.use_pen) {
    hipLaunchKernelGGL((chunk_kernel<DT, true>), grid, dim3(kWave), 0, st, p);
  } else {
    hipLaunchKernelGGL((chunk_kernel<DT, false>), grid, dim3(kWave), 0, st, p);
  }
  if constexpr (MODE == kModeSpec) {
    const int64_t wgs_row = groups * (p.k + 1);
    if (wgs_row > static_cast<int64_t>(device_cu_count())) {
      hipLaunchKernelGGL((spec_row_kernel<DT, 4>), dim3(static_cast<unsigned>(wgs_row)), dim3(kRB), 0, st, p);
    } else {
      hipLaunchKernelGGL((spec_row_kernel<DT, 0>), dim3(static_cast<unsigned>(wgs_row)), dim3(kRB), 0, st, p);
    }
  } else {
    hipLaunchKernelGGL((row_kernel<DT, MODE>), dim3(static_cast<unsigned>(rows)), dim3(kRB), 0, st, p);
  }
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
