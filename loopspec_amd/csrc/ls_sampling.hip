// (a) logit processing and (c) lossless speculative sampling for gfx950.
//
// One 1024-lane workgroup owns one row of logits. The row stays in VGPRs
// (16-byte loads, up to 16 vectors per lane), so HBM is read exactly once:
//
//   1. penalty bitmap of the row's token history in LDS (if penalty != 1);
//   2. x = penalised logits * RN(1/T); m = max x;
//   3. e = ls_exp(x - m), exact fixed-point normaliser S (sum of fx46(e)),
//      and a lane-private octave histogram of e in LDS (conflict-free
//      ds_add_u32 on byte counters);
//   4. top-p: the histogram gives the shallowest octave K whose estimated
//      mass reaches top_p * S; the few elements at or above it are compacted,
//      in index order, into LDS; if their exact mass is short of top_p the
//      next octave is added; an exact 3-round radix select on
//      the binary32 bits of p = e / S with fixed-point masses finds the cutoff
//      c = max{v : sum_{p >= v} fx46(p) >= fx46(top_p)}. The result is valid for
//      the whole row iff c exceeds an upper bound of p outside the candidates;
//      otherwise (or on LDS overflow) a slow path repeats the select over the
//      whole register-resident row. This replaces the reference's full-vocab
//      sort + cumsum + searchsorted (distributions.py:59-70).
//   5. epilogue per mode:
//      - spec:   publish row stats and the support {p >= c} (index order) with
//                device-coherent stores, arrive on the batch element's counter;
//                the last of its 2k+1 rows runs the chain verify (accept tests,
//                residual or bonus draw) for the element;
//      - sample: draw one token from the filtered distribution;
//      - dense:  write p and/or the filtered, renormalised distribution.
//
// All arithmetic is the declared arithmetic of ls_numerics.hpp, so outputs
// are bit-identical to oracle/sampling.py.
#include "ls_common.hpp"
#include "ls_numerics.hpp"
#include "ls_runtime.hpp"

namespace ls {
namespace {

constexpr int kRB = 1024;               // lanes per row workgroup
constexpr int kRW = kRB / kWave;        // waves per row workgroup
constexpr int kBuckets = 16;
constexpr int kCandCap = 2048;          // LDS candidate capacity per row
constexpr int kSupCap = 2048;           // support entries per row in the workspace
constexpr int kMaxNV = 16;              // vectors per lane (row <= 16*1024*16 bytes)
constexpr int kBitmapWords = kMaxNV * kRB * 8 / 32;  // enough bits for the largest row

enum Mode : int { kModeSpec = 0, kModeSample = 1, kModeDense = 2 };
enum RowFlag : uint32_t { kFlagUnfiltered = 1u, kFlagDense = 2u, kFlagSlow = 4u };

// Published per-row statistics (written with device-coherent stores).
struct RowStat {
  float m;          // max processed logit
  float s;          // binary32 normaliser
  float cutoff;     // top-p cutoff value (unused when unfiltered)
  float mass;       // binary32 retained mass (renormaliser)
  uint32_t n_sup;   // support entries published
  uint32_t flags;
  uint64_t s_fx;    // exact normaliser
  uint64_t mass_fx; // exact retained mass
};
static_assert(sizeof(RowStat) == 40, "RowStat layout");

struct SampParams {
  const char* base0;  // target / row logits
  int64_t bstride0, pstride0;  // bytes
  const char* base1;  // draft logits (spec mode)
  int64_t bstride1, pstride1;
  int64_t rows;
  int vocab;
  int nvec;           // 16-byte vectors per row
  int k;              // spec: draft positions; rows per element = 2k+1
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
  RowStat* stats;
  uint64_t* support;            // [rows, kSupCap] of (idx << 32 | bits(p))
  uint32_t* counters;           // [B]
};

// ---------------------------------------------------------------------------
// Device-coherent publication helpers (see ls_common.hpp for the protocol).
// ---------------------------------------------------------------------------
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

// ---------------------------------------------------------------------------
// Block scans (1024 lanes).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t x, int lane) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint64_t y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  return x;
}
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t x, int lane) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  return x;
}

// Exclusive scan in lane order; *total receives the block sum. smem >= kRW+1.
__device__ __forceinline__ uint64_t block_excl_scan_u64(uint64_t v, uint64_t* smem, uint64_t* total) {
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

// ---------------------------------------------------------------------------
// Row context: register-resident row and its processed values.
// ---------------------------------------------------------------------------
struct Shared {
  uint32_t hist[kRW][4][kWave];   // 16 KB; reused as the 2048-entry u64 radix histogram
  uint32_t bitmap[kBitmapWords];  // 16 KB penalty bitmap
  uint32_t cidx[kCandCap];        // candidate / support indices
  float cval[kCandCap];           // candidate e, then p
  uint64_t red[kRW + 2];
  float redf[kRW + 2];
  int base[kMaxNV][kRW];          // compaction offsets per (vector slot, wave)
  int counts[kBuckets];
  uint32_t u32s[8];
  uint64_t u64s[8];
  RowStat st[2 * 64 + 1];         // tail: stats of the element's rows
  int tail_flag;
};

// Per-element logit transform (penalty, temperature); passed by value so no
// helper ever needs the address of the kernel-argument block.
struct Xf {
  float inv_t, pen, inv_pen;
  int use_t, use_pen;
};

__device__ __forceinline__ Xf make_xf(const SampParams& p) {
  return Xf{p.inv_t, p.pen, p.inv_pen, p.use_t, p.use_pen};
}

template <int DT>
__device__ __forceinline__ float xform(const Xf& f, const Shared& sh, float l, int idx) {
  if (f.use_pen) {
    const bool seen = (sh.bitmap[idx >> 5] >> (idx & 31)) & 1u;
    if (seen) l = l < 0.0f ? l * f.pen : l * f.inv_pen;
  }
  if (f.use_t) l = l * f.inv_t;
  return l;
}

// Octave bucket of e when e itself is stored (binary32 exponent) or when only
// the exp's scaling exponent k is known.
__device__ __forceinline__ int bucket_of_e(float e) {
  const int b = 127 - static_cast<int>((__float_as_uint(e) >> 23) & 0xffu);
  return b < kBuckets - 1 ? b : kBuckets - 1;
}
__device__ __forceinline__ int bucket_of_k(int k) {
  if (k == kExpNoBucket) return kBuckets - 1;
  const int b = -k;
  return b < kBuckets - 1 ? b : kBuckets - 1;
}

template <int DT, int NV>
struct Row {
  static constexpr int EPV = Elem<DT>::kPerVec;
  static constexpr bool kStoreE = DT == F32;  // fp32 rows keep e in place of x
  u32x4 d[NV];
  int nvec;
  float m;
  float s;
  uint64_t s_fx;

  __device__ __forceinline__ bool valid(int j) const { return j * kRB + static_cast<int>(threadIdx.x) < nvec; }
  __device__ __forceinline__ int index(int j, int e) const { return (j * kRB + static_cast<int>(threadIdx.x)) * EPV + e; }
  __device__ __forceinline__ float raw(int j, int e) const { return vec_elem<DT>(d[j], e); }
  // e_i for element (j, e): stored or recomputed.
  __device__ __forceinline__ float ev(const Xf& f, const Shared& sh, int j, int e) const {
    if constexpr (kStoreE) {
      return __uint_as_float(d[j][e]);
    } else {
      return ls_exp(xform<DT>(f, sh, raw(j, e), index(j, e)) - m);
    }
  }
};

// ---------------------------------------------------------------------------
// Order-preserving compaction of register elements satisfying pred(j, e)
// into sh.cidx / sh.cval (value from val(j, e)). Element order is the row's
// index order: vector slot j major, then lane, then element within a vector.
// Returns the total count (entries beyond kCandCap are dropped).
// ---------------------------------------------------------------------------
template <int NV, int EPV, typename Pred, typename Val>
__device__ int compact_rows(Shared& sh, Pred pred, Val val) {
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  // EPV mask bits per vector slot, packed 32/EPV slots per word.
  constexpr int kPer = 32 / EPV;
  constexpr int kWords = (NV + kPer - 1) / kPer;
  uint32_t masks[kWords];
#pragma unroll
  for (int q = 0; q < kWords; ++q) masks[q] = 0u;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    uint32_t mk = 0;
#pragma unroll
    for (int e = 0; e < EPV; ++e) mk |= pred(j, e) ? (1u << e) : 0u;
    masks[j / kPer] |= mk << ((j % kPer) * EPV);
    const uint32_t c = __builtin_popcount(mk);
    int tot = 0;
    if (__ballot(c != 0)) tot = __shfl(static_cast<int>(wave_incl_scan_u32(c, lane)), kWave - 1);
    if (lane == 0) sh.base[j][wid] = tot;
  }
  __syncthreads();
  if (wid == 0) {
    // Exclusive scan of the NV*kRW (slot, wave) totals in slot-major order:
    // lane l owns entries [4l, 4l+4).
    constexpr int kE = NV * kRW;
    int* flat = &sh.base[0][0];
    int v[4];
    int local = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i = 4 * lane + q;
      v[q] = i < kE ? flat[i] : 0;
      local += v[q];
    }
    const uint32_t inc = wave_incl_scan_u32(static_cast<uint32_t>(local), lane);
    int run = static_cast<int>(inc) - local;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i = 4 * lane + q;
      if (i < kE) flat[i] = run;
      run += v[q];
    }
    if (lane == kWave - 1) sh.u32s[0] = inc;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const uint32_t mk = (masks[j / kPer] >> ((j % kPer) * EPV)) & ((1u << EPV) - 1u);
    const uint32_t c = __builtin_popcount(mk);
    if (__ballot(c != 0)) {  // rare: recompute this slot's wave offsets
      const uint32_t inc = wave_incl_scan_u32(c, lane);
      int pos = sh.base[j][wid] + static_cast<int>(inc - c);
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        if (mk & (1u << e)) {
          if (pos < kCandCap) {
            sh.cidx[pos] = static_cast<uint32_t>((j * kRB + static_cast<int>(threadIdx.x)) * EPV + e);
            sh.cval[pos] = val(j, e);
          }
          ++pos;
        }
      }
    }
  }
  __syncthreads();
  return static_cast<int>(sh.u32s[0]);
}

// ---------------------------------------------------------------------------
// Exact top-p select: 3 radix rounds (11, 11, 10 bits) over binary32 p bits
// with fixed-point masses. visit(f) calls f(bits, w) for every element of the
// set. Returns false if the set's total mass is below thr.
// ---------------------------------------------------------------------------
template <typename Visit>
__device__ bool radix_select(Shared& sh, uint64_t thr, Visit visit, float* cutoff, uint64_t* mass) {
  uint64_t* H = reinterpret_cast<uint64_t*>(&sh.hist[0][0][0]);
  uint32_t prefix = 0, pmask = 0;
  uint64_t above = 0;
  const int t = threadIdx.x;
  for (int round = 0; round < 3; ++round) {
    const int shift = round == 0 ? 21 : (round == 1 ? 10 : 0);
    const int nbits = round == 2 ? 10 : 11;
    const uint32_t dmask = (1u << nbits) - 1u;
    H[2 * t] = 0;
    H[2 * t + 1] = 0;
    if (t == 0) {
      sh.u32s[1] = 0xffffffffu;
    }
    __syncthreads();
    visit([&](uint32_t bits, uint64_t w) {
      if ((bits & pmask) == prefix && w) {
        __hip_atomic_fetch_add(&H[(bits >> shift) & dmask], w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    });
    __syncthreads();
    // Lane t owns digits hi = 2047-2t and lo = 2046-2t (descending order).
    const int hi = 2047 - 2 * t, lo = 2046 - 2 * t;
    const uint64_t a = hi <= static_cast<int>(dmask) ? H[hi] : 0;
    const uint64_t b = lo <= static_cast<int>(dmask) ? H[lo] : 0;
    uint64_t total;
    const uint64_t ex = block_excl_scan_u64(a + b, sh.red, &total);
    const uint64_t before = above + ex;
    if (before < thr) {
      if (before + a >= thr) {
        sh.u32s[1] = static_cast<uint32_t>(hi);
        sh.u64s[1] = before;
        sh.u64s[2] = a;
      } else if (before + a + b >= thr) {
        sh.u32s[1] = static_cast<uint32_t>(lo);
        sh.u64s[1] = before + a;
        sh.u64s[2] = b;
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

// ---------------------------------------------------------------------------
// Index-ordered inverse-CDF pick over `n` LDS entries (cidx, weight w(i)).
// Lane t owns entries [2t, 2t+2). Returns the chosen index (valid on all
// lanes); zero total mass selects index `zero_index`.
// ---------------------------------------------------------------------------
template <typename W>
__device__ int64_t pick_lds(Shared& sh, int n, float u, W weight, int64_t zero_index) {
  const int t = threadIdx.x;
  const int i0 = 2 * t, i1 = 2 * t + 1;
  const uint64_t w0 = i0 < n ? weight(i0) : 0;
  const uint64_t w1 = i1 < n ? weight(i1) : 0;
  uint64_t total;
  const uint64_t ex = block_excl_scan_u64(w0 + w1, sh.red, &total);
  if (t == 0) sh.u64s[3] = static_cast<uint64_t>(zero_index);
  __syncthreads();
  if (total > 0) {
    const uint64_t target = floor_u_times(u, total);
    if (ex <= target && target < ex + w0 + w1) {
      sh.u64s[3] = sh.cidx[target < ex + w0 ? i0 : i1];
    }
  }
  __syncthreads();
  return static_cast<int64_t>(sh.u64s[3]);
}

// ---------------------------------------------------------------------------
// Dense inverse-CDF pick over a whole row whose weights are computed by
// w(idx) in [0, 1]. Lane t owns a contiguous index range.
// ---------------------------------------------------------------------------
template <typename W>
__device__ int64_t pick_dense(Shared& sh, int vocab, float u, W weight) {
  const int t = threadIdx.x;
  const int per = (vocab + kRB - 1) / kRB;
  const int a = t * per < vocab ? t * per : vocab;
  const int b = a + per < vocab ? a + per : vocab;
  double acc = 0.0;
  uint64_t sum = 0;
  int cnt = 0;
  for (int i = a; i < b; ++i) {
    acc += static_cast<double>(weight(i));
    if (++cnt == 100) {
      sum += static_cast<uint64_t>(acc);
      acc = 0.0;
      cnt = 0;
    }
  }
  sum += static_cast<uint64_t>(acc);
  uint64_t total;
  const uint64_t ex = block_excl_scan_u64(sum, sh.red, &total);
  if (t == 0) sh.u64s[3] = 0;
  __syncthreads();
  if (total > 0) {
    const uint64_t target = floor_u_times(u, total);
    if (ex <= target && target < ex + sum) {
      uint64_t run = ex;
      for (int i = a; i < b; ++i) {
        run += static_cast<uint64_t>(weight(i));
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

// Probability of token `idx` of a published row: recomputed from its logit.
template <int DT>
__device__ float prob_at(const Xf& f, const Shared& sh, const char* row, const RowStat& st, int idx) {
  const float x = xform<DT>(f, sh, load_elem<DT>(row, idx), idx);
  const float pe = ls_exp(x - st.m) / st.s;
  if (st.flags & kFlagUnfiltered) return pe;
  return pe >= st.cutoff ? pe / st.mass : 0.0f;
}

__device__ __forceinline__ const char* row_of(const SampParams& p, int64_t r, int64_t* group) {
  if (p.k > 0) {
    const int rpg = 2 * p.k + 1;
    const int64_t g = r / rpg;
    const int j = static_cast<int>(r - g * rpg);
    *group = g;
    if (j <= p.k) return p.base0 + g * p.bstride0 + j * p.pstride0;
    return p.base1 + g * p.bstride1 + (j - p.k - 1) * p.pstride1;
  }
  *group = r;
  return p.base0 + r * p.pstride0;
}

// ---------------------------------------------------------------------------
// The chain-verify tail for batch element g (whole workgroup, uniform flow).
// ---------------------------------------------------------------------------
template <int DT>
__device__ void spec_tail(const SampParams& p, Shared& sh, int64_t g) {
  const Xf xf = make_xf(p);
  const int k = p.k;
  const int rpg = 2 * k + 1;
  const int t = threadIdx.x;
  if (t < rpg) sh.st[t] = get_stat(p.stats + g * rpg + t);
  if (t == 0) {
    int a = 0;
    while (a < k) {
      const int64_t x = p.draft_tokens[g * k + a];
      const char* trow = p.base0 + g * p.bstride0 + a * p.pstride0;
      const char* drow = p.base1 + g * p.bstride1 + a * p.pstride1;
      bool ok = x >= 0 && x < p.vocab;
      if (ok) {
        // stats are in LDS only after the barrier below; read them directly.
        const RowStat st_t = get_stat(p.stats + g * rpg + a);
        const RowStat st_d = get_stat(p.stats + g * rpg + k + 1 + a);
        const float pt = prob_at<DT>(xf, sh, trow, st_t, static_cast<int>(x));
        const float pd = prob_at<DT>(xf, sh, drow, st_d, static_cast<int>(x));
        ok = accept_draw(p.uniforms[g * rpg + a], pt, pd);
      }
      if (!ok) break;
      p.tokens[g * (k + 1) + a] = x;
      ++a;
    }
    sh.tail_flag = a;
  }
  __syncthreads();
  const int a = sh.tail_flag;
  const RowStat st_t = sh.st[a];
  const char* trow = p.base0 + g * p.bstride0 + a * p.pstride0;
  int64_t token;
  if (a < k) {
    const RowStat st_d = sh.st[k + 1 + a];
    const char* drow = p.base1 + g * p.bstride1 + a * p.pstride1;
    const float u = p.uniforms[g * rpg + k + a];
    const bool sparse = !(st_t.flags & kFlagDense);
    const int n = static_cast<int>(st_t.n_sup);
    const uint64_t* sup = p.support + (g * rpg + a) * static_cast<int64_t>(kSupCap);
    if (sparse) {
      // Support entries of the target row: P_j = p_j / M; Q_j recomputed from
      // the draft logits. D_j = max(P_j - Q_j, 0).
      for (int i = t; i < n; i += kRB) {
        const uint64_t en = load_sc64(sup + i);
        const uint32_t idx = static_cast<uint32_t>(en >> 32);
        const float pj = __uint_as_float(static_cast<uint32_t>(en)) / st_t.mass;
        const float qj = prob_at<DT>(xf, sh, drow, st_d, static_cast<int>(idx));
        const float dj = pj - qj;
        sh.cidx[i] = idx;
        sh.cval[i] = dj > 0.0f ? dj : 0.0f;
        sh.hist[0][0][i] = __float_as_uint(pj);  // keep P_j for the fallback
      }
      __syncthreads();
      uint64_t dsum = 0, psum = 0;
      for (int i = t; i < n; i += kRB) {
        dsum += fx46(sh.cval[i]);
        psum += fx46(__uint_as_float(sh.hist[0][0][i]));
      }
      const uint64_t d_fx = block_sum_u64<kRB>(dsum, sh.red);
      const uint64_t p_fx = block_sum_u64<kRB>(psum, sh.red);
      const bool use_d = d_fx > 0;
      const float den = use_d ? mass_to_f32(d_fx) : (p_fx > 0 ? mass_to_f32(p_fx) : 1.0f);
      token = pick_lds(sh, n, u, [&](int i) {
        const float v = use_d ? sh.cval[i] : __uint_as_float(sh.hist[0][0][i]);
        return fx46(v / den);
      }, 0);
    } else {
      uint64_t dsum = 0, psum = 0;
      {
        const int per = (p.vocab + kRB - 1) / kRB;
        const int i0 = t * per < p.vocab ? t * per : p.vocab;
        const int i1 = i0 + per < p.vocab ? i0 + per : p.vocab;
        double dacc = 0, pacc = 0;
        int c = 0;
        for (int i = i0; i < i1; ++i) {
          const float pj = prob_at<DT>(xf, sh, trow, st_t, i);
          const float qj = prob_at<DT>(xf, sh, drow, st_d, i);
          const float dj = pj - qj;
          dacc += fx46_d(dj > 0.0f ? dj : 0.0f);
          pacc += fx46_d(pj);
          if (++c == 100) {
            dsum += static_cast<uint64_t>(dacc);
            psum += static_cast<uint64_t>(pacc);
            dacc = pacc = 0;
            c = 0;
          }
        }
        dsum += static_cast<uint64_t>(dacc);
        psum += static_cast<uint64_t>(pacc);
      }
      const uint64_t d_fx = block_sum_u64<kRB>(dsum, sh.red);
      const uint64_t p_fx = block_sum_u64<kRB>(psum, sh.red);
      const bool use_d = d_fx > 0;
      const float den = use_d ? mass_to_f32(d_fx) : (p_fx > 0 ? mass_to_f32(p_fx) : 1.0f);
      token = pick_dense(sh, p.vocab, u, [&](int i) {
        const float pj = prob_at<DT>(xf, sh, trow, st_t, i);
        float v = pj;
        if (use_d) {
          const float dj = pj - prob_at<DT>(xf, sh, drow, st_d, i);
          v = dj > 0.0f ? dj : 0.0f;
        }
        return fx46(v / den);
      });
    }
  } else {
    const float u = p.uniforms[g * rpg + 2 * k];
    if (!(st_t.flags & kFlagDense)) {
      const int n = static_cast<int>(st_t.n_sup);
      const uint64_t* sup = p.support + (g * rpg + k) * static_cast<int64_t>(kSupCap);
      for (int i = t; i < n; i += kRB) {
        const uint64_t en = load_sc64(sup + i);
        sh.cidx[i] = static_cast<uint32_t>(en >> 32);
        sh.cval[i] = __uint_as_float(static_cast<uint32_t>(en)) / st_t.mass;
      }
      __syncthreads();
      token = pick_lds(sh, n, u, [&](int i) { return fx46(sh.cval[i]); }, 0);
    } else {
      token = pick_dense(sh, p.vocab, u, [&](int i) { return fx46(prob_at<DT>(xf, sh, trow, st_t, i)); });
    }
  }
  if (t == 0) {
    p.tokens[g * (k + 1) + a] = token;
    for (int j = a + 1; j <= k; ++j) p.tokens[g * (k + 1) + j] = -1;
    p.accept_len[g] = a;
    atomic_exchange_u32(p.counters + g, 0u);
  }
}

// ---------------------------------------------------------------------------
// Slow path of the top-p select: the candidate octave did not hold the cutoff
// (or overflowed LDS). Exact select over every element of the row, re-read
// from memory (it is still cache-resident), then the support {p >= c} is
// compacted in index order; a support larger than kSupCap marks the row dense.
// Kept out of line so the fast path's register allocation is unaffected.
// ---------------------------------------------------------------------------
template <int DT, int NV>
__device__ __noinline__ void slow_select(Xf f, Shared& sh, const char* rowp, int nvec, float m, float s,
                                         uint64_t thr, float* cutoff, uint64_t* mass_fx, int* n_sup,
                                         uint32_t* flags) {
  constexpr int EPV = Elem<DT>::kPerVec;
  const int t = threadIdx.x;
  const u32x4* src = reinterpret_cast<const u32x4*>(rowp);
  auto valid = [&](int j) { return j * kRB + t < nvec; };
  auto pval = [&](int j, int e) -> float {
    const u32x4 d = src[j * kRB + t];
    const int idx = (j * kRB + t) * EPV + e;
    return ls_exp(xform<DT>(f, sh, vec_elem<DT>(d, e), idx) - m) / s;
  };
  float c;
  uint64_t mfx;
  const bool ok = radix_select(sh, thr, [&](auto f) {
    for (int j = 0; j < NV; ++j) {
      if (valid(j)) {
#pragma unroll
        for (int e = 0; e < EPV; ++e) {
          const float pv = pval(j, e);
          f(__float_as_uint(pv), fx46(pv));
        }
      }
    }
  }, &c, &mfx);
  if (ok) {
    *cutoff = c;
    *mass_fx = mfx;
  } else {
    // Total mass below the threshold: the reference clamps to the last sorted
    // value, i.e. keeps the whole row (cutoff = min p).
    float mn = __builtin_inff();
    double acc = 0.0;
    uint64_t tot = 0;
    for (int j = 0; j < NV; ++j) {
      if (valid(j)) {
#pragma unroll
        for (int e = 0; e < EPV; ++e) {
          const float pv = pval(j, e);
          mn = fminf(mn, pv);
          acc += fx46_d(pv);
        }
      }
      tot += static_cast<uint64_t>(acc);
      acc = 0.0;
    }
    *cutoff = -block_max_f32<kRB>(-mn, sh.redf);
    *mass_fx = block_sum_u64<kRB>(tot, sh.red);
  }
  const float cc = *cutoff;
  const int n = compact_rows<NV, EPV>(
      sh, [&](int j, int e) { return valid(j) && pval(j, e) >= cc; }, [&](int j, int e) { return pval(j, e); });
  if (n <= kCandCap && n <= kSupCap) {
    *n_sup = n;
  } else {
    *flags |= kFlagDense;
  }
}

// ---------------------------------------------------------------------------
// The row kernel.
// ---------------------------------------------------------------------------
template <int DT, int NV, int MODE>
__global__ __launch_bounds__(kRB) void sample_rows_kernel(const SampParams p) {
  __shared__ Shared sh;
  using R = Row<DT, NV>;
  constexpr int EPV = R::EPV;
  const int t = threadIdx.x, lane = t & (kWave - 1), wid = t / kWave;
  const int64_t r = blockIdx.x;
  int64_t g;
  const char* rowp = row_of(p, r, &g);
  R row;
  row.nvec = p.nvec;
  const Xf xf = make_xf(p);

  // 1. penalty bitmap (group's history)
  if (p.use_pen) {
    const int words = (p.vocab + 31) >> 5;
    for (int w = t; w < words; w += kRB) sh.bitmap[w] = 0u;
    __syncthreads();
    const int n = p.hist_len ? p.hist_len[g] : 0;
    const int32_t* h = p.hist + g * p.hist_stride;
    for (int i = t; i < n; i += kRB) {
      const int id = h[i];
      if (static_cast<unsigned>(id) < static_cast<unsigned>(p.vocab))
        __hip_atomic_fetch_or(&sh.bitmap[id >> 5], 1u << (id & 31), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }
  // 2. loads (clamped addresses; lanes past the row end re-read its last vector)
  const u32x4* src = reinterpret_cast<const u32x4*>(rowp);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int v = j * kRB + t;
    row.d[j] = __builtin_nontemporal_load(src + (v < p.nvec ? v : p.nvec - 1));
  }
  // zero the lane-private histogram while the loads are in flight
#pragma unroll
  for (int q = 0; q < 4; ++q) sh.hist[wid][q][lane] = 0u;
  __syncthreads();

  // 3. max
  float mx = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    if (row.valid(j)) {
#pragma unroll
      for (int e = 0; e < EPV; ++e) mx = nmax(mx, xform<DT>(xf, sh, row.raw(j, e), row.index(j, e)));
    }
  }
  row.m = block_max_f32<kRB>(mx, sh.redf);

  // 4. exp, exact normaliser, octave histogram
  double sacc = 0.0;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    if (row.valid(j)) {
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        int kexp;
        const float ev = ls_exp_k(xform<DT>(xf, sh, row.raw(j, e), row.index(j, e)) - row.m, &kexp);
        sacc += fx46_d(ev);
        const int b = R::kStoreE ? bucket_of_e(ev) : bucket_of_k(kexp);
        __hip_atomic_fetch_add(&sh.hist[wid][b >> 2][lane], 1u << ((b & 3) * 8), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
        if constexpr (R::kStoreE) row.d[j][e] = __float_as_uint(ev);
      }
    } else if constexpr (R::kStoreE) {
      row.d[j] = u32x4{0u, 0u, 0u, 0u};
    }
  }
  row.s_fx = block_sum_u64<kRB>(static_cast<uint64_t>(sacc), sh.red);
  row.s = mass_to_f32(row.s_fx);

  // histogram totals: widen the byte counters of this lane, reduce per wave,
  // then across waves.
  {
    uint32_t wv[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t w = sh.hist[wid][q][lane];
      wv[2 * q] = w & 0x00ff00ffu;
      wv[2 * q + 1] = (w >> 8) & 0x00ff00ffu;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
#pragma unroll
      for (int q = 0; q < 8; ++q) wv[q] += __shfl_xor(wv[q], o);
    __syncthreads();
    uint32_t* wsum = &sh.hist[0][0][0] + 2048;  // scratch after the first 8 KB
    if (lane == 0)
#pragma unroll
      for (int q = 0; q < 8; ++q) wsum[wid * 8 + q] = wv[q];
    __syncthreads();
    if (t < kBuckets) {
      // bucket b = 4q + s: word q, byte s -> widened word 2q + (s & 1), half s >> 1
      const int q = t >> 2, s = t & 3;
      const int word = 2 * q + (s & 1);
      const int sh16 = (s >> 1) * 16;
      int c = 0;
      for (int w = 0; w < kRW; ++w) c += static_cast<int>((wsum[w * 8 + word] >> sh16) & 0xffffu);
      sh.counts[t] = c;
    }
    __syncthreads();
  }

  const float top_p = p.top_p_rows ? p.top_p_rows[r] : p.top_p;
  const bool unfiltered = !(top_p < 1.0f);
  float cutoff = 0.0f;
  uint64_t mass_fx = row.s_fx;
  uint32_t flags = unfiltered ? (kFlagUnfiltered | kFlagDense) : 0u;
  int n_sup = 0;

  if (!unfiltered) {
    const uint64_t thr = fx46(top_p);
    // 5. candidate octave K: first octave where an estimate of the mass at or
    // above it reaches top_p * S, counting each element of octave b as
    // est * 2^-b (tuned on the benchmark rows so that one attempt suffices:
    // 1.25 when buckets are e's binary exponent, 0.9 for exp-scaling buckets).
    // The estimate only picks where to look; correctness is checked below and
    // K is deepened one octave per failed attempt.
    const double need = static_cast<double>(top_p) * static_cast<double>(row.s);
    const double est = R::kStoreE ? 1.25 : 0.9;
    double cum = 0.0;
    int K = kBuckets - 2;
    for (int b = 0; b < kBuckets - 1; ++b) {
      cum += static_cast<double>(sh.counts[b]) * est * __builtin_ldexp(1.0, -b);
      if (cum >= need) {
        K = b;
        break;
      }
    }
    bool done = false;
    for (int attempt = 0; attempt < 4 && !done && K <= kBuckets - 2; ++attempt, ++K) {
      int ncand = 0;
      for (int b = 0; b <= K; ++b) ncand += sh.counts[b];
      if (ncand > kCandCap) break;
      // 6. compact candidates (bucket <= K) in index order. Only a cheap raw
      // value is stored (e, or t = x - m when e is not kept), so nothing costly
      // is evaluated for the non-candidates; p = e / S is formed afterwards
      // over the compacted entries.
      const uint32_t ebits = __float_as_uint(__builtin_ldexpf(1.0f, -K));
      int n;
      if constexpr (R::kStoreE) {
        n = compact_rows<NV, EPV>(
            sh, [&](int j, int e) { return row.valid(j) && row.d[j][e] >= ebits; },
            [&](int j, int e) { return __uint_as_float(row.d[j][e]); });
      } else {
        const int kk = K;
        n = compact_rows<NV, EPV>(
            sh,
            [&](int j, int e) {
              if (!row.valid(j)) return false;
              const float tt = xform<DT>(xf, sh, row.raw(j, e), row.index(j, e)) - row.m;
              if (!(tt >= kExpMin)) return false;
              return __builtin_rintf(tt * kLog2e) >= static_cast<float>(-kk);
            },
            [&](int j, int e) { return xform<DT>(xf, sh, row.raw(j, e), row.index(j, e)) - row.m; });
      }
      if (n > kCandCap) break;
      for (int i = t; i < n; i += kRB) {
        const float raw = sh.cval[i];
        sh.cval[i] = (R::kStoreE ? raw : ls_exp(raw)) / row.s;
      }
      __syncthreads();
      // exact mass of the candidates; below the threshold -> look one octave deeper
      uint64_t cm = 0;
      for (int i = t; i < n; i += kRB) cm += fx46(sh.cval[i]);
      cm = block_sum_u64<kRB>(cm, sh.red);
      if (cm < thr) continue;
      // 7. exact select among candidates
      float c;
      uint64_t mfx;
      const bool ok = radix_select(sh, thr, [&](auto f) {
        for (int i = t; i < n; i += kRB) {
          const float pv = sh.cval[i];
          f(__float_as_uint(pv), fx46(pv));
        }
      }, &c, &mfx);
      // valid for the row iff c exceeds every p outside the candidates
      const float e_out = R::kStoreE ? __builtin_ldexpf(1.0f, -K) : __builtin_ldexpf(kExpPolyMax, -(K + 1));
      const float p_bound = e_out / row.s;
      if (!(ok && c > p_bound)) continue;
      cutoff = c;
      mass_fx = mfx;
      // support = candidates with p >= c, kept in index order in LDS
      const int i0 = 2 * t, i1 = 2 * t + 1;
      const bool f0 = i0 < n && sh.cval[i0] >= c;
      const bool f1 = i1 < n && sh.cval[i1] >= c;
      const uint32_t x0 = i0 < n ? sh.cidx[i0] : 0u, x1 = i1 < n ? sh.cidx[i1] : 0u;
      const float v0 = i0 < n ? sh.cval[i0] : 0.0f, v1 = i1 < n ? sh.cval[i1] : 0.0f;
      uint64_t tot;
      const uint64_t ex = block_excl_scan_u64(static_cast<uint64_t>(f0) + static_cast<uint64_t>(f1), sh.red, &tot);
      __syncthreads();
      int pos = static_cast<int>(ex);
      if (f0) {
        sh.cidx[pos] = x0;
        sh.cval[pos] = v0;
        ++pos;
      }
      if (f1) {
        sh.cidx[pos] = x1;
        sh.cval[pos] = v1;
      }
      __syncthreads();
      n_sup = static_cast<int>(tot);
      done = true;
    }
    if (!done) {
      // Slow path: exact select over the whole row, re-streamed from memory.
      flags |= kFlagSlow;
      slow_select<DT, NV>(xf, sh, rowp, p.nvec, row.m, row.s, thr, &cutoff, &mass_fx, &n_sup, &flags);
    }
  }
  const float mass = unfiltered ? 1.0f : mass_to_f32(mass_fx);

  if constexpr (MODE == kModeSpec) {
    // 8. publish, arrive; the last row of the element runs the chain tail.
    RowStat st;
    st.m = row.m;
    st.s = row.s;
    st.cutoff = cutoff;
    st.mass = mass;
    st.n_sup = static_cast<uint32_t>(n_sup);
    st.flags = flags;
    st.s_fx = row.s_fx;
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
      const uint32_t prev = atomic_arrive(p.counters + g);
      sh.tail_flag = prev == static_cast<uint32_t>(2 * p.k);
    }
    __syncthreads();
    if (sh.tail_flag) {
      __syncthreads();
      spec_tail<DT>(p, sh, g);
    }
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
        const float x = xform<DT>(xf, sh, load_elem<DT>(rowp, i), i);
        const float pe = ls_exp(x - row.m) / row.s;
        return fx46(unf ? pe : (pe >= cc ? pe / mass : 0.0f));
      });
    }
    if (t == 0) p.row_tokens[r] = token;
  } else {
    // dense outputs
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      if (row.valid(j)) {
#pragma unroll
        for (int e = 0; e < EPV; ++e) {
          const int idx = row.index(j, e);
          if (idx < p.vocab) {
            const float pe = row.ev(xf, sh, j, e) / row.s;
            if (p.probs_out) p.probs_out[r * p.probs_stride + idx] = pe;
            if (p.filt_out)
              p.filt_out[r * p.filt_stride + idx] = unfiltered ? pe : (pe >= cutoff ? pe / mass : 0.0f);
          }
        }
      }
    }
    if (t == 0) {
      if (p.cutoff_out) p.cutoff_out[r] = unfiltered ? 0.0f : cutoff;
      if (p.mass_out) p.mass_out[r] = mass;
    }
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
int nv_for(int nvec) {
  const int need = (nvec + kRB - 1) / kRB;
  const int opts[] = {4, 8, 12, 16};
  for (int o : opts)
    if (need <= o) return o;
  return 0;
}

template <int DT, int MODE>
int launch_nv(const SampParams& p, int nv, int64_t grid, hipStream_t st) {
  const dim3 g(static_cast<unsigned>(grid)), b(kRB);
  switch (nv) {
    case 4: hipLaunchKernelGGL((sample_rows_kernel<DT, 4, MODE>), g, b, 0, st, p); break;
    case 8: hipLaunchKernelGGL((sample_rows_kernel<DT, 8, MODE>), g, b, 0, st, p); break;
    case 12: hipLaunchKernelGGL((sample_rows_kernel<DT, 12, MODE>), g, b, 0, st, p); break;
    case 16: hipLaunchKernelGGL((sample_rows_kernel<DT, 16, MODE>), g, b, 0, st, p); break;
    default: return fail(LS_ERR_VALUE, "vocabulary too large for the register-resident row kernel");
  }
  return check_launch("sampling row kernel launch");
}

template <int MODE>
int launch_mode(const SampParams& p, int dtype, int64_t grid, hipStream_t st) {
  const int nv = nv_for(p.nvec);
  if (nv == 0) return fail(LS_ERR_VALUE, "vocabulary too large for the register-resident row kernel");
  switch (dtype) {
    case LS_DTYPE_F32: return launch_nv<F32, MODE>(p, nv, grid, st);
    case LS_DTYPE_BF16: return launch_nv<BF16, MODE>(p, nv, grid, st);
    case LS_DTYPE_F16: return launch_nv<F16, MODE>(p, nv, grid, st);
    default: return fail(LS_ERR_VALUE, "unsupported logits dtype");
  }
}

// Shared argument validation / setup for the processing options.
int setup_common(SampParams& p, int dtype, int64_t vocab, float temperature, float top_p, int64_t top_k,
                 float penalty, const int32_t* history, int64_t history_stride, const int32_t* history_len) {
  const int eb = dtype_bytes(dtype);
  if (eb == 0) return fail(LS_ERR_VALUE, "unsupported logits dtype");
  if (vocab <= 0 || vocab > (1 << 24)) return fail(LS_ERR_VALUE, "invalid vocabulary size");
  if ((vocab * eb) % 16 != 0) return fail(LS_ERR_VALUE, "vocabulary row bytes must be a multiple of 16");
  if (!(temperature > 0.0f)) return fail(LS_ERR_VALUE, "temperature must be > 0");
  if (!(top_p > 0.0f) || top_p > 1.0f) return fail(LS_ERR_VALUE, "top_p must be in (0, 1]");
  if (top_k != 0 && top_k < vocab) return fail(LS_ERR_VALUE, "top_k filtering is not supported by this entry point");
  if (!(penalty > 0.0f)) return fail(LS_ERR_VALUE, "repetition penalty must be > 0");
  if (penalty != 1.0f && (history == nullptr || history_len == nullptr))
    return fail(LS_ERR_VALUE, "repetition penalty needs a token history");
  p.vocab = static_cast<int>(vocab);
  p.nvec = static_cast<int>(vocab * eb / 16);
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

// Workspace layout. The arrival counters sit at a fixed offset (0) with room
// for kMaxSpecBatch elements: they are the only words that must be zero when
// a launch starts, and a fixed place keeps them clear of the stats/support
// regions of a previous call with another (batch, k) on the same buffer.
constexpr int64_t kMaxSpecBatch = 16384;

uint64_t spec_ws_layout(int64_t batch, int64_t k, uint64_t* off_stats, uint64_t* off_sup, uint64_t* off_cnt) {
  const int64_t rows = batch * (2 * k + 1);
  const uint64_t cnt = static_cast<uint64_t>(kMaxSpecBatch) * 4ull;
  const uint64_t stats = (static_cast<uint64_t>(rows) * sizeof(RowStat) + 255) & ~255ull;
  const uint64_t sup = static_cast<uint64_t>(rows) * kSupCap * 8ull;
  *off_cnt = 0;
  *off_stats = cnt;
  *off_sup = cnt + stats;
  return cnt + stats + sup;
}

}  // namespace
}  // namespace ls

using namespace ls;

extern "C" {

uint64_t ls_spec_verify_workspace(int64_t batch, int64_t k, int64_t vocab) {
  (void)vocab;
  if (batch <= 0 || k < 1) return 0;
  uint64_t a, b, c;
  return spec_ws_layout(batch, k, &a, &b, &c);
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
  p.rows = batch * (2 * k + 1);
  p.draft_tokens = draft_tokens;
  p.uniforms = uniforms;
  p.accept_len = accept_len;
  p.tokens = tokens;
  uint64_t o_st, o_sup, o_cnt;
  const uint64_t need = spec_ws_layout(batch, k, &o_st, &o_sup, &o_cnt);
  if (!workspace || ws_bytes < need) return fail(LS_ERR_VALUE, "spec_verify: workspace too small");
  char* ws = static_cast<char*>(workspace);
  p.stats = reinterpret_cast<RowStat*>(ws + o_st);
  p.support = reinterpret_cast<uint64_t*>(ws + o_sup);
  p.counters = reinterpret_cast<uint32_t*>(ws + o_cnt);
  return launch_mode<kModeSpec>(p, dtype, p.rows, static_cast<hipStream_t>(stream));
}

int ls_sample_logits(const void* logits, int64_t row_stride, int dtype, int64_t rows, int64_t vocab,
                     float temperature, float top_p, int64_t top_k, float penalty, const int32_t* history,
                     int64_t history_stride, const int32_t* history_len, const float* uniforms,
                     int64_t* out_tokens, ls_stream_t stream) {
  if (rows < 0) return fail(LS_ERR_VALUE, "sample_logits: invalid rows");
  if (rows == 0) return LS_OK;
  if (!logits || !uniforms || !out_tokens) return fail(LS_ERR_VALUE, "sample_logits: NULL pointer");
  SampParams p{};
  int rc = setup_common(p, dtype, vocab, temperature, top_p, top_k, penalty, history, history_stride, history_len);
  if (rc) return rc;
  const int eb = dtype_bytes(dtype);
  p.base0 = static_cast<const char*>(logits);
  p.pstride0 = row_stride * eb;
  if (!aligned16(logits) || p.pstride0 % 16) return fail(LS_ERR_VALUE, "sample_logits: rows must be 16-byte aligned");
  p.rows = rows;
  p.row_uniforms = uniforms;
  p.row_tokens = out_tokens;
  return launch_mode<kModeSample>(p, dtype, rows, static_cast<hipStream_t>(stream));
}

int ls_filter_logits(const void* logits, int64_t row_stride, int dtype, int64_t rows, int64_t vocab,
                     float temperature, float top_p, const float* top_p_rows, int64_t top_k, float* probs_out,
                     int64_t probs_stride, float* filtered_out, int64_t filtered_stride, float* cutoff_out,
                     float* mass_out, ls_stream_t stream) {
  if (rows < 0) return fail(LS_ERR_VALUE, "filter_logits: invalid rows");
  if (rows == 0) return LS_OK;
  if (!logits) return fail(LS_ERR_VALUE, "filter_logits: NULL logits");
  SampParams p{};
  int rc = setup_common(p, dtype, vocab, temperature, top_p, top_k, 1.0f, nullptr, 0, nullptr);
  if (rc) return rc;
  const int eb = dtype_bytes(dtype);
  p.base0 = static_cast<const char*>(logits);
  p.pstride0 = row_stride * eb;
  if (!aligned16(logits) || p.pstride0 % 16) return fail(LS_ERR_VALUE, "filter_logits: rows must be 16-byte aligned");
  p.rows = rows;
  p.top_p_rows = top_p < 1.0f ? top_p_rows : nullptr;
  p.probs_out = probs_out;
  p.probs_stride = probs_stride;
  p.filt_out = filtered_out;
  p.filt_stride = filtered_stride;
  p.cutoff_out = cutoff_out;
  p.mass_out = mass_out;
  return launch_mode<kModeDense>(p, dtype, rows, static_cast<hipStream_t>(stream));
}

}  // extern "C"
