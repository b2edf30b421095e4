// (a) logit processing and (c) lossless speculative sampling for gfx950.
//
// The logits are read once, by many workgroups per row. The declared softmax
// is chunked (kChunk elements per chunk; see oracle/sampling.py): everything a
// chunk needs depends only on the chunk, and the row-wide values combine the
// chunks' results exactly. Two or three launches per call, stream-ordered:
//
//   chunk_kernel  one 256-lane workgroup per (row, chunk): penalty bits of
//                 the chunk's index range, x = pen(l) * RN(1/T), chunk max m_j,
//                 e = ls_exp(x - m_j), exact chunk mass M_j = sum fx46(e), an
//                 octave histogram of e, and the chunk's largest entries (all
//                 e >= 2^(1-K_j), at most kChunkCand, K_j from the histogram)
//                 compacted in index order into the workspace. No
//                 cross-workgroup communication.
//   row_kernel    one 1024-lane workgroup per row: m = max m_j,
//                 f_j = ls_exp(m_j - m), S from the exact sum of f_j * M_j,
//                 p = RN(RN(e f_j) / S) for the candidates, exact top-p cutoff
//                 by a 3-round radix select on the binary32 bits of p with
//                 fixed-point masses (replacing sort + cumsum + searchsorted,
//                 distributions.py:59-70), valid for the whole row iff it
//                 exceeds every p outside the candidates (else an exact select
//                 over the re-streamed row). Then per mode:
//                   spec   publish the row's stats and support {p >= c} with
//                          device-coherent stores and arrive on the batch
//                          element's counter; the last of its 2k+1 rows runs
//                          the chain verify (accept tests, residual / bonus
//                          draw);
//                   sample draw one token from the filtered distribution;
//                   dense  publish the row's stats for dense_kernel.
//   dense_kernel  (dense mode) one workgroup per (row, chunk) writes p and/or
//                 the filtered, renormalised distribution.
//
// All arithmetic is the declared arithmetic of ls_numerics.hpp, so every
// output is bit-identical to the oracle's.
#include "ls_common.hpp"
#include "ls_numerics.hpp"
#include "ls_runtime.hpp"

namespace ls {
namespace {

constexpr int kChunk = 8192;                 // softmax chunk (declared arithmetic)
constexpr int kCB = 256;                     // chunk kernel lanes
constexpr int kCW = kCB / kWave;
constexpr int kChunkCand = 256;              // candidates kept per chunk (at most)
constexpr int kOct = 64;                     // octave bins of e
constexpr int kRB = 512;                     // row kernel lanes
constexpr int kRW = kRB / kWave;
constexpr int kRowCand = 4096;               // candidates of a row held in LDS
constexpr int kMaxChunks = 32;               // vocab <= 262144
constexpr int kMaxVocab = kMaxChunks * kChunk;
constexpr int kSupCap = 2048;                // support entries per row in the workspace
constexpr int kBins = 2048;                  // radix digits per round
constexpr int kBinsPerLane = kBins / kRB;
constexpr int kCounterStride = 16;           // arrival counters one 64-byte line apart
constexpr int kChunkWgsPerCu = 3;            // persistent chunk workgroups per CU
constexpr int64_t kMaxSpecBatch = 16384;
constexpr int64_t kMaxGridYZ = 65535;

enum Mode : int { kModeSpec = 0, kModeSample = 1, kModeDense = 2 };
enum RowFlag : uint32_t { kFlagUnfiltered = 1u, kFlagDense = 2u, kFlagSlow = 4u };
enum ChunkFlag : uint32_t { kChunkComplete = 1u };

// Per-chunk result of chunk_kernel.
struct ChunkRec {
  float m;          // chunk max of the processed logits
  int32_t K;        // candidates are the e >= 2^(1-K) (all e > 0 when complete)
  uint32_t n;       // candidates written
  uint32_t flags;
  uint64_t mass;    // exact chunk mass sum fx46(e)
  uint64_t pad;
};
static_assert(sizeof(ChunkRec) == 32, "ChunkRec layout");

// Published per-row statistics.
struct RowStat {
  float m;          // row max of the processed logits
  float s;          // binary32 normaliser
  float cutoff;     // top-p cutoff value (0 when unfiltered)
  float mass;       // binary32 retained mass (renormaliser)
  uint32_t n_sup;   // support entries published
  uint32_t flags;
  uint64_t s_fx;    // exact normaliser
  uint64_t mass_fx; // exact retained mass
};
static_assert(sizeof(RowStat) == 40, "RowStat layout");

struct SampParams {
  const char* base0;           // target / row logits
  int64_t bstride0, pstride0;  // bytes
  const char* base1;           // draft logits (spec mode)
  int64_t bstride1, pstride1;
  int rpg;                     // rows per group: spec 2k+1, else 1
  int k;                       // spec: draft positions; 0 otherwise
  int vocab;
  int nch;                     // chunks per row
  int chunk_cap;               // candidates kept per chunk: min(kChunkCand, kRowCand / nch)
  int bm_words;                // penalty bitmap words per group (0 without penalty)
  float inv_t;
  int use_t;
  float pen, inv_pen;
  int use_pen;
  float top_p;                 // >= 1: unfiltered
  const float* top_p_rows;     // optional per-row top_p (dense/sample modes)
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
  uint64_t* support;            // [rows, kSupCap] of (idx << 32 | bits(p)) (spec)
  uint32_t* counters;           // [kMaxSpecBatch * kCounterStride] (spec)
  uint32_t* bitmap;             // [groups, bm_words] penalty bits (written by chunk_kernel)
};

// Row jr of group g: spec rows are target positions 0..k, then draft 0..k-1.
__device__ __forceinline__ const char* row_of(const SampParams& p, int64_t g, int jr) {
  if (jr <= p.k) return p.base0 + g * p.bstride0 + jr * p.pstride0;
  return p.base1 + g * p.bstride1 + (jr - p.k - 1) * p.pstride1;
}

// Per-element logit transform (penalty, temperature); passed by value so no
// helper needs the address of the kernel-argument block.
struct Xf {
  float inv_t, pen, inv_pen;
  int use_t, use_pen;
};

__device__ __forceinline__ Xf make_xf(const SampParams& p) {
  return Xf{p.inv_t, p.pen, p.inv_pen, p.use_t, p.use_pen};
}

__device__ __forceinline__ float xform_seen(const Xf& f, float l, bool seen) {
  if (f.use_pen && seen) l = l < 0.0f ? l * f.pen : l * f.inv_pen;
  if (f.use_t) l = l * f.inv_t;
  return l;
}

__device__ __forceinline__ bool bit_of(const uint32_t* bm, int idx) { return (bm[idx >> 5] >> (idx & 31)) & 1u; }

// p of one element from its chunk max m_j, the row max m and the normaliser s.
__device__ __forceinline__ float chunk_p(float x, float mj, float m, float s) {
  const float e = ls_exp(x - mj);
  const float f = ls_exp(mj - m);
  return (e * f) / s;
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
// chunk_kernel
// ===========================================================================
struct ChunkShared {
  uint32_t oct[kCW][kOct];             // per-wave octave counts
  float wmax[kCW];
  uint64_t wmass[kCW];
  int wcnt[8][kCW];                    // candidates per (vector slot, wave)
};

// Inclusive wave scan of a 32-bit value (DPP).
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t x, int lane) {
  (void)lane;
  return wave_scan_add_u32(x);
}

// Loads of one chunk (clamped: lanes past the chunk end re-read its last
// vector), plus, with a penalty, the bitmap word of each vector (the EPV bits
// of a 16-byte vector always sit in one 32-bit word).
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
    const int v = u * kCB + static_cast<int>(threadIdx.x);
    d[u] = __builtin_nontemporal_load(src + (v < nvc ? v : nvc - 1));
  }
  if (p.use_pen) {
    const uint32_t* bm = p.bitmap + static_cast<int64_t>(g) * p.bm_words + c0 / 32;
#pragma unroll
    for (int u = 0; u < NVC; ++u) pw[u] = bm[((u * kCB + static_cast<int>(threadIdx.x)) * EPV) >> 5];
  }
}

// One chunk. Three barriers: after the chunk max, after the mass / histogram
// (every wave then derives K on its own), after the per-(slot, wave)
// candidate counts (every wave then derives its output offsets on its own).
// The LDS of the previous chunk is safe to reuse without a barrier: every
// read of it precedes a barrier that each wave passes before the writes here.
template <int DT, int NVC>
__device__ __forceinline__ void process_chunk(const SampParams& p, ChunkShared& sh, int item, const u32x4 (&d)[NVC],
                                              const uint32_t (&pw)[NVC]) {
  constexpr int EPV = Elem<DT>::kPerVec;
  constexpr int NE = NVC * EPV;  // 32 elements per lane
  const int t = threadIdx.x, lane = t & (kWave - 1), wid = t / kWave;
  const int r = item / p.nch;
  const int cj = item - r * p.nch;
  const int g = r / p.rpg;
  const int jr = r - g * p.rpg;
  const int c0 = cj * kChunk;
  const int nel = p.vocab - c0 < kChunk ? p.vocab - c0 : kChunk;
  const int nvc = nel / EPV;
  const Xf xf = make_xf(p);
  sh.oct[wid][lane] = 0u;
  // 3. processed logits x (kept as binary32 bit patterns) and the chunk max
  uint32_t xe[NE];
  float mx = -__builtin_inff();
  const bool full = nvc == kCB * NVC;  // only a row's last chunk can be partial
  if (xf.use_pen | xf.use_t) {
#pragma unroll
    for (int u = 0; u < NVC; ++u) {
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        const bool seen = xf.use_pen && ((pw[u] >> ((((u * kCB + t) * EPV) & 31) + e)) & 1u);
        xe[u * EPV + e] = __float_as_uint(xform_seen(xf, vec_elem<DT>(d[u], e), seen));
      }
    }
  } else {
#pragma unroll
    for (int u = 0; u < NVC; ++u) {
#pragma unroll
      for (int e = 0; e < EPV; ++e) xe[u * EPV + e] = __float_as_uint(vec_elem<DT>(d[u], e));
    }
  }
  if (!full) {
#pragma unroll
    for (int u = 0; u < NVC; ++u) {
      if (u * kCB + t >= nvc) {
#pragma unroll
        for (int e = 0; e < EPV; ++e) xe[u * EPV + e] = 0xff800000u;  // -inf
      }
    }
  }
#pragma unroll
  for (int i = 0; i < NE; i += 2) mx = nmax(mx, nmax(__uint_as_float(xe[i]), __uint_as_float(xe[i + 1])));
  mx = wave_max_f32(mx);
  if (lane == 0) sh.wmax[wid] = mx;
  __syncthreads();
  const float m = nmax(nmax(sh.wmax[0], sh.wmax[1]), nmax(sh.wmax[2], sh.wmax[3]));
  // 4. e in place, exact chunk mass (integer fx46), octave histogram. Every
  // element is counted (e == 0 in the last bin), which only matters for
  // K == 64 and keeps the loop branch-free.
  uint64_t acc = 0;
#pragma unroll
  for (int i = 0; i < NE; ++i) {
    const uint32_t b = __float_as_uint(ls_exp(__uint_as_float(xe[i]) - m));  // -inf / NaN give 0
    xe[i] = b;
    const uint32_t E = b >> 23;
    const uint32_t sh_r = 127u - E;
    const uint64_t mant = static_cast<uint64_t>((b & 0x7fffffu) | 0x800000u) << 23;
    acc += sh_r > 47u ? 0ull : (mant >> sh_r);  // floor(e * 2^46), exact
    const uint32_t o = sh_r < static_cast<uint32_t>(kOct - 1) ? sh_r : static_cast<uint32_t>(kOct - 1);
    __hip_atomic_fetch_add(&sh.oct[wid][o], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  const uint64_t wm = wave_sum_u64(acc);
  if (lane == 0) sh.wmass[wid] = wm;
  __syncthreads();
  // 5. K (every wave): the largest number of leading octaves holding at most
  // chunk_cap entries.
  int K;
  {
    uint32_t c = 0;
#pragma unroll
    for (int w = 0; w < kCW; ++w) c += sh.oct[w][lane];
    const uint32_t inc = wave_scan_u32(c, lane);
    K = __builtin_popcountll(__ballot(inc <= static_cast<uint32_t>(p.chunk_cap)));
  }
  // e qualifies iff e >= 2^(1-K) (K == 64: every e > 0; K == 0: none)
  const uint32_t thr_bits = K >= kOct ? 1u : (K == 0 ? 0x7f800000u : static_cast<uint32_t>(128 - K) << 23);
  // 6. candidate counts per (vector slot, wave); index order is (slot, lane, e)
  uint32_t cs[NVC];
#pragma unroll
  for (int u = 0; u < NVC; ++u) {
    uint32_t c = 0;
#pragma unroll
    for (int e = 0; e < EPV; ++e) c += xe[u * EPV + e] >= thr_bits ? 1u : 0u;
    cs[u] = c;
    int tot = 0;
    if (__ballot(c != 0)) tot = static_cast<int>(lane_bcast_u32(wave_scan_u32(c, lane), kWave - 1));
    if (lane == 0) sh.wcnt[u][wid] = tot;
  }
  __syncthreads();
  // 7. this wave's base offset per slot: exclusive prefix over (slot, wave)
  // in slot-major order, computed by every wave from the shared counts.
  int flat = 0;
  if (lane < NVC * kCW) flat = sh.wcnt[lane / kCW][lane % kCW];
  const int incl = static_cast<int>(wave_scan_u32(static_cast<uint32_t>(flat), lane));
  const int total = static_cast<int>(lane_bcast_u32(static_cast<uint32_t>(incl), NVC * kCW - 1));
  uint64_t* out = p.cands + (static_cast<int64_t>(r) * p.nch + cj) * kChunkCand;
  const int cap = p.chunk_cap;
#pragma unroll
  for (int u = 0; u < NVC; ++u) {
    const uint32_t c = cs[u];
    if (__ballot(c != 0)) {
      const int slot = u * kCW + wid;
      const int base = static_cast<int>(lane_bcast_u32(static_cast<uint32_t>(incl), slot) -
                                        lane_bcast_u32(static_cast<uint32_t>(flat), slot));
      int pos = base + static_cast<int>(wave_scan_u32(c, lane) - c);
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        if (xe[u * EPV + e] >= thr_bits) {
          if (pos < cap) {
            const uint32_t idx = static_cast<uint32_t>(c0 + (u * kCB + t) * EPV + e);
            out[pos] = (static_cast<uint64_t>(idx) << 32) | xe[u * EPV + e];
          }
          ++pos;
        }
      }
    }
  }
  if (t == 0) {
    ChunkRec rec;
    rec.m = m;
    rec.K = K;
    rec.n = static_cast<uint32_t>(total < cap ? total : cap);
    rec.flags = K >= kOct ? kChunkComplete : 0u;
    rec.mass = sh.wmass[0] + sh.wmass[1] + sh.wmass[2] + sh.wmass[3];
    rec.pad = 0;
    p.chunks[static_cast<int64_t>(r) * p.nch + cj] = rec;
  }
}

// Persistent over (row, chunk) items in row-major order, double-buffered: the
// next item's loads are in flight while the current one is processed.
template <int DT>
__global__ __launch_bounds__(kCB, 3) void chunk_kernel(const SampParams p, int items) {
  constexpr int EPV = Elem<DT>::kPerVec;
  constexpr int NVC = kChunk / (kCB * EPV);  // vectors per lane: 8 (f32) or 4
  __shared__ ChunkShared sh;
  int item = blockIdx.x;
  if (item >= items) return;
  u32x4 cur[NVC], nxt[NVC];
  uint32_t pcur[NVC] = {}, pnxt[NVC] = {};
  load_chunk<DT, NVC>(p, item, cur, pcur);
  while (true) {
    const int next = item + static_cast<int>(gridDim.x);
    if (next < items) load_chunk<DT, NVC>(p, next, nxt, pnxt);
    process_chunk<DT, NVC>(p, sh, item, cur, pcur);
    if (next >= items) break;
#pragma unroll
    for (int u = 0; u < NVC; ++u) {
      cur[u] = nxt[u];
      pcur[u] = pnxt[u];
    }
    item = next;
  }
}

// ===========================================================================
// row_kernel
// ===========================================================================
struct RowShared {
  uint32_t cidx[kRowCand];       // candidate / support indices
  float cval[kRowCand];          // candidate / support p
  uint64_t H[kBins];             // radix histogram
  float pa[128];                 // tail: P and Q of the draft tokens
  uint32_t gbits[kWave];         // select: entries of the cutoff's bucket
  uint64_t gw[kWave];
  int gcount;
  float cm[kMaxChunks], cf[kMaxChunks];
  int cK[kMaxChunks], coff[kMaxChunks + 1];
  uint32_t cn[kMaxChunks], cfl[kMaxChunks];
  uint64_t cM[kMaxChunks];
  uint64_t red[kRW + 2];
  float redf[kRW + 2];
  uint32_t u32s[8];
  uint64_t u64s[8];
  RowStat st[2 * 64 + 1];        // tail: stats of the element's rows
  int tail_flag;
};

__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t x, int lane) {
  (void)lane;
  return wave_scan_add_u64(x);
}

// Exclusive scan in lane order over the 1024 lanes; *total receives the sum.
__device__ __forceinline__ uint64_t row_excl_scan(uint64_t v, uint64_t* smem, uint64_t* total) {
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  const uint64_t inc = wave_incl_scan_u64(v, lane);
  __syncthreads();
  if (lane == kWave - 1) smem[wid] = inc;
  __syncthreads();
  uint64_t base = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kRW; ++i) {
    const uint64_t s = smem[i];
    base += i < wid ? s : 0;
    tot += s;
  }
  *total = tot;
  return base + inc - v;
}

// Exact top-p select: 3 radix rounds (11, 11, 10 bits) over binary32 p bits
// with fixed-point masses. visit(f) calls f(bits, w) for every element of the
// set. Returns false if the set's total mass is below thr.
template <typename Visit>
__device__ bool radix_select(RowShared& sh, uint64_t thr, Visit visit, float* cutoff, uint64_t* mass) {
  uint64_t* H = sh.H;
  uint32_t prefix = 0, pmask = 0;
  uint64_t above = 0;
  const int t = threadIdx.x;
  for (int round = 0; round < 3; ++round) {
    const int shift = round == 0 ? 21 : (round == 1 ? 10 : 0);
    const int nbits = round == 2 ? 10 : 11;
    const uint32_t dmask = (1u << nbits) - 1u;
#pragma unroll
    for (int q = 0; q < kBinsPerLane; ++q) H[kBinsPerLane * t + q] = 0;
    if (t == 0) sh.u32s[1] = 0xffffffffu;
    __syncthreads();
    visit([&](uint32_t bits, uint64_t w) {
      if ((bits & pmask) == prefix && w) {
        __hip_atomic_fetch_add(&H[(bits >> shift) & dmask], w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    });
    __syncthreads();
    // Lane t owns digits kBins-1 - (kBinsPerLane*t + q), q = 0.. (descending).
    uint64_t v[kBinsPerLane];
    uint64_t sum = 0;
#pragma unroll
    for (int q = 0; q < kBinsPerLane; ++q) {
      const int dg = kBins - 1 - (kBinsPerLane * t + q);
      v[q] = dg <= static_cast<int>(dmask) ? H[dg] : 0;
      sum += v[q];
    }
    uint64_t total;
    const uint64_t ex = row_excl_scan(sum, sh.red, &total);
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
    __syncthreads();
    const uint32_t digit = sh.u32s[1];
    if (digit == 0xffffffffu) return false;
    prefix |= digit << shift;
    pmask |= dmask << shift;
    above = sh.u64s[1];
    if (round == 2) {
      *cutoff = __uint_as_float(prefix);
      *mass = above + sh.u64s[2];
    }
    __syncthreads();
  }
  return true;
}

// Exact cutoff over the n LDS candidates (sh.cval): one 11-bit radix round
// on the top bits of p picks the bucket holding the cutoff; a bucket of at
// most 64 entries is finished by one wave (each lane ranks its entry against
// the others), a larger one by the full 3-round select.
__device__ bool select_candidates(RowShared& sh, int n, uint64_t thr, float* cutoff, uint64_t* mass) {
  const int t = threadIdx.x, lane = t & (kWave - 1), wid = t / kWave;
  uint64_t* H = sh.H;
#pragma unroll
  for (int q = 0; q < kBinsPerLane; ++q) H[kBinsPerLane * t + q] = 0;
  if (t == 0) {
    sh.u32s[1] = 0xffffffffu;
    sh.gcount = 0;
  }
  __syncthreads();
  for (int i = t; i < n; i += kRB) {
    const float pv = sh.cval[i];
    const uint64_t w = fx46(pv);
    if (w) __hip_atomic_fetch_add(&H[__float_as_uint(pv) >> 21], w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  __syncthreads();
  {
    uint64_t v[kBinsPerLane];
    uint64_t sum = 0;
#pragma unroll
    for (int q = 0; q < kBinsPerLane; ++q) {
      v[q] = H[kBins - 1 - (kBinsPerLane * t + q)];
      sum += v[q];
    }
    uint64_t total;
    uint64_t before = row_excl_scan(sum, sh.red, &total);
    if (before < thr && before + sum >= thr) {
#pragma unroll
      for (int q = 0; q < kBinsPerLane; ++q) {
        if (before < thr && before + v[q] >= thr) {
          sh.u32s[1] = static_cast<uint32_t>(kBins - 1 - (kBinsPerLane * t + q));
          sh.u64s[1] = before;
        }
        before += v[q];
      }
    }
  }
  __syncthreads();
  const uint32_t d1 = sh.u32s[1];
  if (d1 == 0xffffffffu) return false;
  const uint64_t above = sh.u64s[1];
  for (int i = t; i < n; i += kRB) {
    const float pv = sh.cval[i];
    const uint32_t bits = __float_as_uint(pv);
    const uint64_t w = fx46(pv);
    if ((bits >> 21) == d1 && w) {
      const int k = __hip_atomic_fetch_add(&sh.gcount, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (k < kWave) {
        sh.gbits[k] = bits;
        sh.gw[k] = w;
      }
    }
  }
  __syncthreads();
  const int cnt = sh.gcount;
  if (cnt > kWave) {
    __syncthreads();
    return radix_select(sh, thr, [&](auto f) {
      for (int i = t; i < n; i += kRB) {
        const float pv = sh.cval[i];
        f(__float_as_uint(pv), fx46(pv));
      }
    }, cutoff, mass);
  }
  if (wid == 0) {
    const uint32_t b = lane < cnt ? sh.gbits[lane] : 0u;
    const uint64_t w = lane < cnt ? sh.gw[lane] : 0;
    uint64_t A = above;
    for (int j = 0; j < cnt; ++j) {
      const uint32_t bj = lane_bcast_u32(b, j);
      const uint64_t wj = lane_bcast_u64(w, j);
      A += bj >= b ? wj : 0;
    }
    const bool ok = lane < cnt && A >= thr;
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

// Index-ordered inverse-CDF pick over n LDS entries (cidx, weight w(i)),
// n <= kRowCand; lane t owns entries [8t, 8t+8). Zero total mass selects
// zero_index.
template <typename W>
__device__ int64_t pick_lds(RowShared& sh, int n, float u, W weight, int64_t zero_index) {
  constexpr int kPer = kRowCand / kRB;
  const int t = threadIdx.x;
  const int i0 = kPer * t;
  uint64_t sum = 0;
#pragma unroll
  for (int q = 0; q < kPer; ++q) sum += i0 + q < n ? weight(i0 + q) : 0;
  uint64_t total;
  const uint64_t ex = row_excl_scan(sum, sh.red, &total);
  if (t == 0) sh.u64s[3] = static_cast<uint64_t>(zero_index);
  __syncthreads();
  if (total > 0) {
    const uint64_t target = floor_u_times(u, total);
    if (ex <= target && target < ex + sum) {
      uint64_t run = ex;
      for (int q = 0; q < kPer; ++q) {
        if (i0 + q >= n) break;
        run += weight(i0 + q);
        if (run > target) {
          sh.u64s[3] = sh.cidx[i0 + q];
          break;
        }
      }
    }
  }
  __syncthreads();
  return static_cast<int64_t>(sh.u64s[3]);
}

// Dense inverse-CDF pick over a whole row whose masses are computed by
// weight(idx) (an exact fx46 integer). Lane t owns a contiguous index range.
template <typename W>
__device__ int64_t pick_dense(RowShared& sh, int vocab, float u, W weight) {
  const int t = threadIdx.x;
  const int per = (vocab + kRB - 1) / kRB;
  const int a = t * per < vocab ? t * per : vocab;
  const int b = a + per < vocab ? a + per : vocab;
  uint64_t sum = 0;
  for (int i = a; i < b; ++i) sum += weight(i);
  uint64_t total;
  const uint64_t ex = row_excl_scan(sum, sh.red, &total);
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

__device__ __forceinline__ void put_stat(RowStat* st, const RowStat& v) {
  uint32_t* w = reinterpret_cast<uint32_t*>(st);
  store_sc(w + 0, __float_as_uint(v.m));
  store_sc(w + 1, __float_as_uint(v.s));
  store_sc(w + 2, __float_as_uint(v.cutoff));
  store_sc(w + 3, __float_as_uint(v.mass));
  store_sc(w + 4, v.n_sup);
  store_sc(w + 5, v.flags);
  store_sc64(reinterpret_cast<uint64_t*>(w + 6), v.s_fx);
  store_sc64(reinterpret_cast<uint64_t*>(w + 8), v.mass_fx);
}
__device__ __forceinline__ RowStat get_stat(const RowStat* st) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(st);
  RowStat v;
  v.m = __uint_as_float(load_sc(w + 0));
  v.s = __uint_as_float(load_sc(w + 1));
  v.cutoff = __uint_as_float(load_sc(w + 2));
  v.mass = __uint_as_float(load_sc(w + 3));
  v.n_sup = load_sc(w + 4);
  v.flags = load_sc(w + 5);
  v.s_fx = load_sc64(reinterpret_cast<const uint64_t*>(w + 6));
  v.mass_fx = load_sc64(reinterpret_cast<const uint64_t*>(w + 8));
  return v;
}

// Filtered probability of token idx of row r (stats st), recomputed from its
// logit; bm is the group's penalty bitmap.
template <int DT>
__device__ float prob_at(const SampParams& p, const Xf& f, const uint32_t* bm, int64_t r, const char* rowp,
                         const RowStat& st, int idx) {
  const float x = xform_seen(f, load_elem<DT>(rowp, idx), f.use_pen && bit_of(bm, idx));
  const float mj = p.chunks[r * p.nch + (idx / kChunk)].m;
  const float pe = chunk_p(x, mj, st.m, st.s);
  if (st.flags & kFlagUnfiltered) return pe;
  return pe >= st.cutoff ? pe / st.mass : 0.0f;
}

// The chain-verify tail for batch element g (whole workgroup, uniform flow).
template <int DT>
__device__ void spec_tail(const SampParams& p, RowShared& sh, int64_t g, const uint32_t* bm) {
  const Xf xf = make_xf(p);
  const int k = p.k;
  const int rpg = 2 * k + 1;
  const int t = threadIdx.x;
  const int64_t r0 = g * rpg;
  if (t < rpg) sh.st[t] = get_stat(p.stats + r0 + t);
  __syncthreads();
  // P_i(x_i) (lanes i < k) and Q_i(x_i) (lanes k + i), all in flight together
  if (t < 2 * k) {
    const int i = t < k ? t : t - k;
    const int jr = t < k ? i : k + 1 + i;
    const int64_t x = p.draft_tokens[g * k + i];
    float v = 0.0f;
    if (x >= 0 && x < p.vocab) v = prob_at<DT>(p, xf, bm, r0 + jr, row_of(p, g, jr), sh.st[jr], static_cast<int>(x));
    sh.pa[t] = v;
  }
  __syncthreads();
  if (t == 0) {
    int a = 0;
    while (a < k) {
      const int64_t x = p.draft_tokens[g * k + a];
      const bool ok = x >= 0 && x < p.vocab && accept_draw(p.uniforms[g * rpg + a], sh.pa[a], sh.pa[k + a]);
      if (!ok) break;
      p.tokens[g * (k + 1) + a] = x;
      ++a;
    }
    sh.tail_flag = a;
  }
  __syncthreads();
  const int a = sh.tail_flag;
  const RowStat st_t = sh.st[a];
  const char* trow = row_of(p, g, a);
  int64_t token;
  if (a < k) {
    const RowStat st_d = sh.st[k + 1 + a];
    const char* drow = row_of(p, g, k + 1 + a);
    const int64_t rt = r0 + a, rd = r0 + k + 1 + a;
    const float u = p.uniforms[g * rpg + k + a];
    if (!(st_t.flags & kFlagDense)) {
      // Support entries of the target row: P_j = p_j / M; Q_j recomputed from
      // the draft logits; D_j = max(P_j - Q_j, 0). P_j is kept in H for the
      // zero-residual fallback.
      const int n = static_cast<int>(st_t.n_sup);
      const uint64_t* sup = p.support + rt * static_cast<int64_t>(kSupCap);
      float* pkeep = reinterpret_cast<float*>(sh.H);
      for (int i = t; i < n; i += kRB) {
        const uint64_t en = load_sc64(sup + i);
        const uint32_t idx = static_cast<uint32_t>(en >> 32);
        const float pj = __uint_as_float(static_cast<uint32_t>(en)) / st_t.mass;
        const float qj = prob_at<DT>(p, xf, bm, rd, drow, st_d, static_cast<int>(idx));
        const float dj = pj - qj;
        sh.cidx[i] = idx;
        sh.cval[i] = dj > 0.0f ? dj : 0.0f;
        pkeep[i] = pj;
      }
      __syncthreads();
      uint64_t dsum = 0, psum = 0;
      for (int i = t; i < n; i += kRB) {
        dsum += fx46(sh.cval[i]);
        psum += fx46(pkeep[i]);
      }
      const uint64_t d_fx = block_sum_u64<kRB>(dsum, sh.red);
      const uint64_t p_fx = block_sum_u64<kRB>(psum, sh.red);
      const bool use_d = d_fx > 0;
      const float den = use_d ? mass_to_f32(d_fx) : (p_fx > 0 ? mass_to_f32(p_fx) : 1.0f);
      token = pick_lds(sh, n, u, [&](int i) {
        const float v = use_d ? sh.cval[i] : pkeep[i];
        return fx46(v / den);
      }, 0);
    } else {
      uint64_t dsum = 0, psum = 0;
      {
        const int per = (p.vocab + kRB - 1) / kRB;
        const int i0 = t * per < p.vocab ? t * per : p.vocab;
        const int i1 = i0 + per < p.vocab ? i0 + per : p.vocab;
        for (int i = i0; i < i1; ++i) {
          const float pj = prob_at<DT>(p, xf, bm, rt, trow, st_t, i);
          const float qj = prob_at<DT>(p, xf, bm, rd, drow, st_d, i);
          const float dj = pj - qj;
          dsum += fx46(dj > 0.0f ? dj : 0.0f);
          psum += fx46(pj);
        }
      }
      const uint64_t d_fx = block_sum_u64<kRB>(dsum, sh.red);
      const uint64_t p_fx = block_sum_u64<kRB>(psum, sh.red);
      const bool use_d = d_fx > 0;
      const float den = use_d ? mass_to_f32(d_fx) : (p_fx > 0 ? mass_to_f32(p_fx) : 1.0f);
      token = pick_dense(sh, p.vocab, u, [&](int i) {
        const float pj = prob_at<DT>(p, xf, bm, rt, trow, st_t, i);
        float v = pj;
        if (use_d) {
          const float dj = pj - prob_at<DT>(p, xf, bm, rd, drow, st_d, i);
          v = dj > 0.0f ? dj : 0.0f;
        }
        return fx46(v / den);
      });
    }
  } else {
    const float u = p.uniforms[g * rpg + 2 * k];
    const int64_t rt = r0 + k;
    if (!(st_t.flags & kFlagDense)) {
      const int n = static_cast<int>(st_t.n_sup);
      const uint64_t* sup = p.support + rt * static_cast<int64_t>(kSupCap);
      for (int i = t; i < n; i += kRB) {
        const uint64_t en = load_sc64(sup + i);
        sh.cidx[i] = static_cast<uint32_t>(en >> 32);
        sh.cval[i] = __uint_as_float(static_cast<uint32_t>(en)) / st_t.mass;
      }
      __syncthreads();
      token = pick_lds(sh, n, u, [&](int i) { return fx46(sh.cval[i]); }, 0);
    } else {
      token = pick_dense(sh, p.vocab, u,
                         [&](int i) { return fx46(prob_at<DT>(p, xf, bm, rt, trow, st_t, i)); });
    }
  }
  if (t == 0) {
    p.tokens[g * (k + 1) + a] = token;
    for (int j = a + 1; j <= k; ++j) p.tokens[g * (k + 1) + j] = -1;
    p.accept_len[g] = a;
    store_sc(p.counters + g * kCounterStride, 0u);
  }
}

// Exact select over every element of the row (the candidates did not hold
// the cutoff): p recomputed from the re-read logits. Leaves the support
// {p >= c} in index order in LDS when it fits, else flags the row dense.
// Kept out of line so the common path's register allocation is unaffected.
template <int DT>
__device__ __noinline__ void slow_select(const SampParams& p, RowShared& sh, const char* rowp, const uint32_t* bm,
                                         float m, float s, uint64_t thr, float* cutoff, uint64_t* mass_fx,
                                         int* n_sup, uint32_t* flags) {
  const Xf xf = make_xf(p);
  const int t = threadIdx.x;
  const int vocab = p.vocab;
  auto pval = [&](int i) -> float {
    const float x = xform_seen(xf, load_elem<DT>(rowp, i), xf.use_pen && bit_of(bm, i));
    return chunk_p(x, sh.cm[i / kChunk], m, s);
  };
  float c;
  uint64_t mfx;
  const bool ok = radix_select(sh, thr, [&](auto f) {
    for (int i = t; i < vocab; i += kRB) {
      const float pv = pval(i);
      f(__float_as_uint(pv), fx46(pv));
    }
  }, &c, &mfx);
  if (ok) {
    *cutoff = c;
    *mass_fx = mfx;
  } else {
    // Total mass below the threshold: keep the whole row (cutoff = min p).
    float mn = __builtin_inff();
    uint64_t tot = 0;
    for (int i = t; i < vocab; i += kRB) {
      const float pv = pval(i);
      mn = fminf(mn, pv);
      tot += fx46(pv);
    }
    *cutoff = -block_max_f32<kRB>(-mn, sh.redf);
    *mass_fx = block_sum_u64<kRB>(tot, sh.red);
  }
  const float cc = *cutoff;
  // support in index order: contiguous lane ranges, counted then written
  const int per = (vocab + kRB - 1) / kRB;
  const int a = t * per < vocab ? t * per : vocab;
  const int b = a + per < vocab ? a + per : vocab;
  uint64_t cnt = 0;
  for (int i = a; i < b; ++i) cnt += pval(i) >= cc ? 1 : 0;
  uint64_t total;
  const uint64_t ex = row_excl_scan(cnt, sh.red, &total);
  if (total <= static_cast<uint64_t>(kSupCap)) {
    int pos = static_cast<int>(ex);
    for (int i = a; i < b; ++i) {
      const float pv = pval(i);
      if (pv >= cc) {
        sh.cidx[pos] = static_cast<uint32_t>(i);
        sh.cval[pos] = pv;
        ++pos;
      }
    }
    *n_sup = static_cast<int>(total);
  } else {
    *flags |= kFlagDense;
  }
  __syncthreads();
}

template <int DT, int MODE>
__global__ __launch_bounds__(kRB, 4) void row_kernel(const SampParams p) {
  __shared__ RowShared sh;
  const int t = threadIdx.x;
  const int jr = blockIdx.x;
  const int64_t g = blockIdx.y;
  const int64_t r = g * p.rpg + jr;
  const char* rowp = row_of(p, g, jr);
  const Xf xf = make_xf(p);
  const int nch = p.nch;

  // chunk records (wave 0: one lane per chunk): m, f_j, T, candidate offsets
  const uint32_t* bm = p.use_pen ? p.bitmap + g * p.bm_words : nullptr;  // group's penalty bits
  if (t < kWave) {
    const int lane = t;
    ChunkRec rec{};
    rec.m = -__builtin_inff();
    if (lane < nch) rec = p.chunks[r * nch + lane];
    const float rm = wave_max_f32(rec.m);
    const float f = lane < nch ? ls_exp(rec.m - rm) : 0.0f;
    const uint64_t T = wave_sum_u64(lane < nch ? floor_u_times(f, rec.mass) : 0);
    const uint32_t cnt = lane < nch ? rec.n : 0u;
    const uint32_t inc = wave_scan_add_u32(cnt);
    if (lane < nch) {
      sh.cm[lane] = rec.m;
      sh.cf[lane] = f;
      sh.cK[lane] = rec.K;
      sh.cn[lane] = rec.n;
      sh.cfl[lane] = rec.flags;
      sh.coff[lane] = static_cast<int>(inc - cnt);
    }
    if (lane == nch - 1) sh.coff[nch] = static_cast<int>(inc);
    if (lane == 0) {
      sh.u64s[0] = T;
      sh.u32s[0] = __float_as_uint(rm);
    }
  }
  __syncthreads();
  const float m = __uint_as_float(sh.u32s[0]);
  const uint64_t s_fx = sh.u64s[0];
  const float s = mass_to_f32(s_fx);

  const float top_p = p.top_p_rows ? p.top_p_rows[r] : p.top_p;
  const bool unfiltered = !(top_p < 1.0f);
  float cutoff = 0.0f;
  uint64_t mass_fx = s_fx;
  uint32_t flags = unfiltered ? (kFlagUnfiltered | kFlagDense) : 0u;
  int n_sup = 0;

  if (!unfiltered) {
    const uint64_t thr = fx46(top_p);
    // candidates of every chunk, p = RN(RN(e f_j) / S), in index order
    const int n = sh.coff[nch];
    for (int i = t; i < n; i += kRB) {
      int j = 0;
      while (j + 1 < nch && sh.coff[j + 1] <= i) ++j;
      const uint64_t en = p.cands[(r * nch + j) * static_cast<int64_t>(kChunkCand) + (i - sh.coff[j])];
      const float e = __uint_as_float(static_cast<uint32_t>(en));
      sh.cidx[i] = static_cast<uint32_t>(en >> 32);
      sh.cval[i] = (e * sh.cf[j]) / s;
    }
    // every p outside the candidates is <= p_bound
    float p_bound = 0.0f;
    for (int j = 0; j < nch; ++j) {
      if (!(sh.cfl[j] & kChunkComplete)) {
        const float eb = __builtin_ldexpf(sh.cf[j], 1 - sh.cK[j]);
        p_bound = fmaxf(p_bound, eb / s);
      }
    }
    __syncthreads();
    float c;
    uint64_t mfx;
    const bool ok = select_candidates(sh, n, thr, &c, &mfx);
    if (ok && c > p_bound) {
      cutoff = c;
      mass_fx = mfx;
      // support = candidates with p >= c, compacted in index order in LDS
      constexpr int kPer = kRowCand / kRB;
      const int i0 = kPer * t;
      uint32_t keep = 0;
      uint64_t cnt = 0;
#pragma unroll
      for (int q = 0; q < kPer; ++q) {
        const bool f = i0 + q < n && sh.cval[i0 + q] >= c;
        keep |= f ? (1u << q) : 0u;
        cnt += f ? 1 : 0;
      }
      uint32_t xi[kPer];
      float xv[kPer];
#pragma unroll
      for (int q = 0; q < kPer; ++q) {
        xi[q] = (keep >> q) & 1u ? sh.cidx[i0 + q] : 0u;
        xv[q] = (keep >> q) & 1u ? sh.cval[i0 + q] : 0.0f;
      }
      uint64_t tot;
      const uint64_t ex = row_excl_scan(cnt, sh.red, &tot);
      __syncthreads();
      int pos = static_cast<int>(ex);
#pragma unroll
      for (int q = 0; q < kPer; ++q) {
        if ((keep >> q) & 1u) {
          sh.cidx[pos] = xi[q];
          sh.cval[pos] = xv[q];
          ++pos;
        }
      }
      __syncthreads();
      n_sup = static_cast<int>(tot);
      if (MODE == kModeSpec && n_sup > kSupCap) flags |= kFlagDense;
    } else {
      flags |= kFlagSlow;
      slow_select<DT>(p, sh, rowp, bm, m, s, thr, &cutoff, &mass_fx, &n_sup, &flags);
    }
  }
  const float mass = unfiltered ? 1.0f : mass_to_f32(mass_fx);

  if constexpr (MODE == kModeSpec) {
    RowStat st;
    st.m = m;
    st.s = s;
    st.cutoff = cutoff;
    st.mass = mass;
    st.n_sup = static_cast<uint32_t>(n_sup);
    st.flags = flags;
    st.s_fx = s_fx;
    st.mass_fx = mass_fx;
    if (!(flags & kFlagDense)) {
      uint64_t* sup = p.support + r * static_cast<int64_t>(kSupCap);
      for (int i = t; i < n_sup; i += kRB)
        store_sc64(sup + i, (static_cast<uint64_t>(sh.cidx[i]) << 32) | __float_as_uint(sh.cval[i]));
    }
    if (t == 0) put_stat(p.stats + r, st);
    drain_stores();
    __syncthreads();
    if (t == 0) {
      const uint32_t prev = atomic_arrive(p.counters + g * kCounterStride);
      sh.tail_flag = prev == static_cast<uint32_t>(p.rpg - 1);
    }
    __syncthreads();
    if (sh.tail_flag) spec_tail<DT>(p, sh, g, bm);
  } else if constexpr (MODE == kModeSample) {
    const float u = p.row_uniforms[r];
    int64_t token;
    if (!(flags & kFlagDense)) {
      const float mf = mass;
      token = pick_lds(sh, n_sup, u, [&](int i) { return fx46(sh.cval[i] / mf); }, 0);
    } else {
      const float cc = cutoff;
      const bool unf = unfiltered;
      token = pick_dense(sh, p.vocab, u, [&](int i) {
        const float x = xform_seen(xf, load_elem<DT>(rowp, i), xf.use_pen && bit_of(bm, i));
        const float pe = chunk_p(x, sh.cm[i / kChunk], m, s);
        return fx46(unf ? pe : (pe >= cc ? pe / mass : 0.0f));
      });
    }
    if (t == 0) p.row_tokens[r] = token;
  } else {
    if (t == 0) {
      RowStat st;
      st.m = m;
      st.s = s;
      st.cutoff = cutoff;
      st.mass = mass;
      st.n_sup = 0;
      st.flags = flags;
      st.s_fx = s_fx;
      st.mass_fx = mass_fx;
      p.stats[r] = st;
      if (p.cutoff_out) p.cutoff_out[r] = unfiltered ? 0.0f : cutoff;
      if (p.mass_out) p.mass_out[r] = mass;
    }
  }
}

// ===========================================================================
// dense_kernel: p and the filtered distribution for one (row, chunk)
// ===========================================================================
template <int DT>
__global__ __launch_bounds__(kCB) void dense_kernel(const SampParams p) {
  constexpr int EPV = Elem<DT>::kPerVec;
  constexpr int NVC = kChunk / (kCB * EPV);
  const int t = threadIdx.x;
  const int cj = blockIdx.x;
  const int64_t r = blockIdx.z;
  const char* rowp = row_of(p, r, 0);
  const int c0 = cj * kChunk;
  const int nel = p.vocab - c0 < kChunk ? p.vocab - c0 : kChunk;
  const int nvc = nel / EPV;
  const u32x4* src = reinterpret_cast<const u32x4*>(rowp) + c0 / EPV;
  const RowStat st = p.stats[r];
  const float mj = p.chunks[r * p.nch + cj].m;
  const float f = ls_exp(mj - st.m);
  const Xf xf = make_xf(p);
  const bool unf = st.flags & kFlagUnfiltered;
#pragma unroll
  for (int u = 0; u < NVC; ++u) {
    const int v = u * kCB + t;
    if (v < nvc) {
      const u32x4 d = __builtin_nontemporal_load(src + v);
      float pv[EPV], fv[EPV];
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        const float x = xform_seen(xf, vec_elem<DT>(d, e), false);
        const float pe = (ls_exp(x - mj) * f) / st.s;
        pv[e] = pe;
        fv[e] = unf ? pe : (pe >= st.cutoff ? pe / st.mass : 0.0f);
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
  uint64_t cnt, chunks, cands, stats, support, bitmap, total;
};

// Workspace: [spec: arrival counters, one 64-byte line each, for up to
// kMaxSpecBatch elements at a fixed place] [chunk records] [candidates]
// [row stats] [spec: supports] [penalty bitmaps, one per group].
Layout ws_layout(int64_t rows, int64_t groups, int nch, bool spec) {
  auto al = [](uint64_t x) { return (x + 255u) & ~255ull; };
  Layout l{};
  l.cnt = 0;
  uint64_t off = spec ? al(static_cast<uint64_t>(kMaxSpecBatch) * kCounterStride * 4u) : 0;
  l.chunks = off;
  off = al(off + static_cast<uint64_t>(rows) * nch * sizeof(ChunkRec));
  l.cands = off;
  off = al(off + static_cast<uint64_t>(rows) * nch * kChunkCand * 8u);
  l.stats = off;
  off = al(off + static_cast<uint64_t>(rows) * sizeof(RowStat));
  l.support = off;
  if (spec) off = al(off + static_cast<uint64_t>(rows) * kSupCap * 8u);
  l.bitmap = off;
  off = al(off + static_cast<uint64_t>(groups) * nch * (kChunk / 32) * 4u);
  l.total = off;
  return l;
}

void bind_workspace(SampParams& p, void* ws, const Layout& l) {
  char* b = static_cast<char*>(ws);
  p.counters = reinterpret_cast<uint32_t*>(b + l.cnt);
  p.chunks = reinterpret_cast<ChunkRec*>(b + l.chunks);
  p.cands = reinterpret_cast<uint64_t*>(b + l.cands);
  p.stats = reinterpret_cast<RowStat*>(b + l.stats);
  p.support = reinterpret_cast<uint64_t*>(b + l.support);
  p.bitmap = reinterpret_cast<uint32_t*>(b + l.bitmap);
}

int nch_for(int64_t vocab) { return static_cast<int>((vocab + kChunk - 1) / kChunk); }

template <int DT, int MODE>
void launch_dt(const SampParams& p, int64_t groups, hipStream_t st) {
  const unsigned gz = static_cast<unsigned>(groups);
  if (p.use_pen) hipLaunchKernelGGL(bitmap_kernel, dim3(gz), dim3(kBmB), 0, st, p);
  const int items = static_cast<int>(groups * p.rpg * p.nch);
  const int wgs = static_cast<int>(device_cu_count()) * kChunkWgsPerCu;
  hipLaunchKernelGGL((chunk_kernel<DT>), dim3(items < wgs ? items : wgs), dim3(kCB), 0, st, p, items);
  hipLaunchKernelGGL((row_kernel<DT, MODE>), dim3(p.rpg, gz), dim3(kRB), 0, st, p);
  if constexpr (MODE == kModeDense) {
    hipLaunchKernelGGL((dense_kernel<DT>), dim3(p.nch, 1, gz), dim3(kCB), 0, st, p);
  }
}

template <int MODE>
int launch_mode(const SampParams& p, int dtype, int64_t groups, hipStream_t st) {
  switch (dtype) {
    case LS_DTYPE_F32: launch_dt<F32, MODE>(p, groups, st); break;
    case LS_DTYPE_BF16: launch_dt<BF16, MODE>(p, groups, st); break;
    case LS_DTYPE_F16: launch_dt<F16, MODE>(p, groups, st); break;
    default: return fail(LS_ERR_VALUE, "unsupported logits dtype");
  }
  return check_launch("sampling kernel launch");
}

// Shared argument validation / setup for the processing options.
int setup_common(SampParams& p, int dtype, int64_t vocab, float temperature, float top_p, int64_t top_k,
                 float penalty, const int32_t* history, int64_t history_stride, const int32_t* history_len) {
  const int eb = dtype_bytes(dtype);
  if (eb == 0) return fail(LS_ERR_VALUE, "unsupported logits dtype");
  if (vocab <= 0 || vocab > kMaxVocab) return fail(LS_ERR_VALUE, "vocabulary size must be in [1, 262144]");
  if ((vocab * eb) % 16 != 0) return fail(LS_ERR_VALUE, "vocabulary row bytes must be a multiple of 16");
  if (!(temperature > 0.0f)) return fail(LS_ERR_VALUE, "temperature must be > 0");
  if (!(top_p > 0.0f) || top_p > 1.0f) return fail(LS_ERR_VALUE, "top_p must be in (0, 1]");
  if (top_k != 0 && top_k < vocab) return fail(LS_ERR_VALUE, "top_k filtering is not supported by this entry point");
  if (!(penalty > 0.0f)) return fail(LS_ERR_VALUE, "repetition penalty must be > 0");
  if (penalty != 1.0f && (history == nullptr || history_len == nullptr))
    return fail(LS_ERR_VALUE, "repetition penalty needs a token history");
  p.vocab = static_cast<int>(vocab);
  p.nch = nch_for(vocab);
  p.chunk_cap = kRowCand / p.nch < kChunkCand ? kRowCand / p.nch : kChunkCand;
  p.bm_words = p.nch * (kChunk / 32);
  p.use_t = temperature != 1.0f;
  p.inv_t = 1.0f / temperature;
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
  return ws_layout(batch * (2 * k + 1), batch, nch_for(vocab), true).total;
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
  int rc = setup_common(p, dtype, vocab, temperature, top_p, top_k, penalty, history, history_stride, history_len);
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
  const Layout l = ws_layout(batch * p.rpg, batch, p.nch, true);
  if (!workspace || ws_bytes < l.total) return fail(LS_ERR_VALUE, "spec_verify: workspace too small");
  bind_workspace(p, workspace, l);
  return launch_mode<kModeSpec>(p, dtype, batch, static_cast<hipStream_t>(stream));
}

uint64_t ls_sample_logits_workspace(int64_t rows, int64_t vocab) {
  if (rows <= 0 || vocab <= 0) return 0;
  return ws_layout(rows, rows, nch_for(vocab), false).total;
}

int ls_sample_logits(const void* logits, int64_t row_stride, int dtype, int64_t rows, int64_t vocab,
                     float temperature, float top_p, int64_t top_k, float penalty, const int32_t* history,
                     int64_t history_stride, const int32_t* history_len, const float* uniforms,
                     int64_t* out_tokens, void* workspace, uint64_t ws_bytes, ls_stream_t stream) {
  if (rows < 0 || rows > kMaxGridYZ) return fail(LS_ERR_VALUE, "sample_logits: need 0 <= rows <= 65535");
  if (rows == 0) return LS_OK;
  if (!logits || !uniforms || !out_tokens) return fail(LS_ERR_VALUE, "sample_logits: NULL pointer");
  SampParams p{};
  int rc = setup_common(p, dtype, vocab, temperature, top_p, top_k, penalty, history, history_stride, history_len);
  if (rc) return rc;
  const int eb = dtype_bytes(dtype);
  p.base0 = static_cast<const char*>(logits);
  p.bstride0 = row_stride * eb;
  if (!aligned16(logits) || p.bstride0 % 16) return fail(LS_ERR_VALUE, "sample_logits: rows must be 16-byte aligned");
  p.rpg = 1;
  p.k = 0;
  p.row_uniforms = uniforms;
  p.row_tokens = out_tokens;
  const Layout l = ws_layout(rows, rows, p.nch, false);
  if (!workspace || ws_bytes < l.total) return fail(LS_ERR_VALUE, "sample_logits: workspace too small");
  bind_workspace(p, workspace, l);
  return launch_mode<kModeSample>(p, dtype, rows, static_cast<hipStream_t>(stream));
}

uint64_t ls_filter_logits_workspace(int64_t rows, int64_t vocab) {
  if (rows <= 0 || vocab <= 0) return 0;
  return ws_layout(rows, rows, nch_for(vocab), false).total;
}

int ls_filter_logits(const void* logits, int64_t row_stride, int dtype, int64_t rows, int64_t vocab,
                     float temperature, float top_p, const float* top_p_rows, int64_t top_k, float* probs_out,
                     int64_t probs_stride, float* filtered_out, int64_t filtered_stride, float* cutoff_out,
                     float* mass_out, void* workspace, uint64_t ws_bytes, ls_stream_t stream) {
  if (rows < 0 || rows > kMaxGridYZ) return fail(LS_ERR_VALUE, "filter_logits: need 0 <= rows <= 65535");
  if (rows == 0) return LS_OK;
  if (!logits) return fail(LS_ERR_VALUE, "filter_logits: NULL logits");
  SampParams p{};
  int rc = setup_common(p, dtype, vocab, temperature, top_p, top_k, 1.0f, nullptr, 0, nullptr);
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
  const Layout l = ws_layout(rows, rows, p.nch, false);
  if (!workspace || ws_bytes < l.total) return fail(LS_ERR_VALUE, "filter_logits: workspace too small");
  bind_workspace(p, workspace, l);
  return launch_mode<kModeDense>(p, dtype, rows, static_cast<hipStream_t>(stream));
}

}  // extern "C"
