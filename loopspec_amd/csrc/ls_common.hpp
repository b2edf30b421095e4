// Shared device helpers for the LoopSpec verify/sample kernels (gfx950, wave64).
//
// Everything here is written for CDNA4 directly: 64-lane wavefronts, LDS for
// cross-wave exchange, agent-scope atomics for the "last workgroup finishes
// the group" pattern used to fuse a cross-row epilogue into one launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ls {

// Logit / probability element types accepted at the C-ABI (matches the codes in
// include/loopspec_hip.h).
enum DType : int { F32 = 0, BF16 = 1, F16 = 2 };

constexpr int kWave = 64;

// Native 16-byte vector (one global_load_dwordx4 per lane).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Element decode. A 16-byte vector holds 4 fp32 or 8 bf16/fp16 values.
// ---------------------------------------------------------------------------
template <int DT> struct Elem;
template <> struct Elem<F32> { static constexpr int kPerVec = 4; static constexpr int kBytes = 4; };
template <> struct Elem<BF16> { static constexpr int kPerVec = 8; static constexpr int kBytes = 2; };
template <> struct Elem<F16> { static constexpr int kPerVec = 8; static constexpr int kBytes = 2; };

__device__ __forceinline__ float f16_bits_to_float(uint32_t h) {
  _Float16 v;
  uint16_t b = static_cast<uint16_t>(h);
  __builtin_memcpy(&v, &b, 2);
  return static_cast<float>(v);
}

// Decode element e (0 <= e < kPerVec) of a 16-byte vector.
template <int DT>
__device__ __forceinline__ float vec_elem(const u32x4& d, int e) {
  if constexpr (DT == F32) {
    return __uint_as_float(d[e]);
  } else if constexpr (DT == BF16) {
    const uint32_t x = d[e >> 1];
    return (e & 1) ? __uint_as_float(x & 0xffff0000u) : __uint_as_float(x << 16);
  } else {
    const uint32_t x = d[e >> 1];
    return f16_bits_to_float((e & 1) ? (x >> 16) : (x & 0xffffu));
  }
}

// Scalar decode of element i of a row (unaligned fallback path).
template <int DT>
__device__ __forceinline__ float load_elem(const void* row, int64_t i) {
  if constexpr (DT == F32) {
    return static_cast<const float*>(row)[i];
  } else if constexpr (DT == BF16) {
    const uint32_t b = static_cast<const uint16_t*>(row)[i];
    return __uint_as_float(b << 16);
  } else {
    return f16_bits_to_float(static_cast<const uint16_t*>(row)[i]);
  }
}

// Element i's storage bits (16-bit types zero-extended by the load itself) and
// their decode, apart: a gather of bits leaves its loads outstanding until the
// decode at the values' use, where a decoding load would wait for them at once.
template <int DT>
__device__ __forceinline__ uint32_t load_bits(const void* row, int64_t i) {
  if constexpr (DT == F32) {
    return static_cast<const uint32_t*>(row)[i];
  } else {
    return static_cast<const uint16_t*>(row)[i];
  }
}

template <int DT>
__device__ __forceinline__ float bits_to_float(uint32_t b) {
  if constexpr (DT == F32) {
    return __uint_as_float(b);
  } else if constexpr (DT == BF16) {
    return __uint_as_float(b << 16);
  } else {
    return f16_bits_to_float(b);
  }
}

// NaN-propagating maximum (IEEE-754 2019 `maximum`); lowers to v_maximum3_f32.
__device__ __forceinline__ float nmax(float a, float b) {
  return __builtin_elementwise_maximum(a, b);
}

// Maximum of all elements of one vector, NaN-propagating.
template <int DT>
__device__ __forceinline__ float vec_max(const u32x4& d) {
  if constexpr (DT == F32) {
    return nmax(nmax(__uint_as_float(d[0]), __uint_as_float(d[1])),
                nmax(__uint_as_float(d[2]), __uint_as_float(d[3])));
  } else {
    float m = vec_elem<DT>(d, 0);
#pragma unroll
    for (int e = 1; e < 8; ++e) m = nmax(m, vec_elem<DT>(d, e));
    return m;
  }
}

// Total order on floats used by argmax: NaN above everything, -0 == +0.
// Larger key == larger value.
__device__ __forceinline__ uint32_t ordered_key(float v) {
  if (v != v) return 0xffffffffu;
  const uint32_t b = __float_as_uint(v) == 0x80000000u ? 0u : __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// (value, index) packed so that unsigned max picks the larger value and, on a
// tie, the lower index -- torch.argmax's rule. Key 0 means "no element".
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
  return (static_cast<uint64_t>(ordered_key(v)) << 32) | static_cast<uint64_t>(0xffffffffu - idx);
}
__device__ __forceinline__ uint32_t argmax_key_index(uint64_t key) {
  return 0xffffffffu - static_cast<uint32_t>(key & 0xffffffffu);
}

// ---------------------------------------------------------------------------
// Wave scans and reductions (wave64) on DPP: row_shr 1, 2, 4, 8 build the
// inclusive scan inside each row of 16 lanes, row_bcast:15 and row_bcast:31
// carry the row totals forward, all in the VALU (a __shfl is an LDS
// ds_bpermute round trip per step). Every lane of the wave must be active.
// Reductions read the scan's last lane.
// ---------------------------------------------------------------------------
constexpr int kDppRowShr1 = 0x111, kDppRowShr2 = 0x112, kDppRowShr4 = 0x114, kDppRowShr8 = 0x118;
constexpr int kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;

template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp32(uint32_t ident, uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(static_cast<int>(ident), static_cast<int>(v), CTRL, ROWS, 0xf, false));
}

template <int CTRL, int ROWS>
__device__ __forceinline__ uint64_t dpp64(uint64_t ident, uint64_t v) {
  const uint32_t lo = dpp32<CTRL, ROWS>(static_cast<uint32_t>(ident), static_cast<uint32_t>(v));
  const uint32_t hi = dpp32<CTRL, ROWS>(static_cast<uint32_t>(ident >> 32), static_cast<uint32_t>(v >> 32));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// Inclusive scans.
__device__ __forceinline__ uint32_t wave_scan_add_u32(uint32_t v) {
  v += dpp32<kDppRowShr1, 0xf>(0u, v);
  v += dpp32<kDppRowShr2, 0xf>(0u, v);
  v += dpp32<kDppRowShr4, 0xf>(0u, v);
  v += dpp32<kDppRowShr8, 0xf>(0u, v);
  v += dpp32<kDppRowBcast15, 0xa>(0u, v);
  v += dpp32<kDppRowBcast31, 0xc>(0u, v);
  return v;
}

__device__ __forceinline__ uint64_t wave_scan_add_u64(uint64_t v) {
  v += dpp64<kDppRowShr1, 0xf>(0ull, v);
  v += dpp64<kDppRowShr2, 0xf>(0ull, v);
  v += dpp64<kDppRowShr4, 0xf>(0ull, v);
  v += dpp64<kDppRowShr8, 0xf>(0ull, v);
  v += dpp64<kDppRowBcast15, 0xa>(0ull, v);
  v += dpp64<kDppRowBcast31, 0xc>(0ull, v);
  return v;
}

__device__ __forceinline__ uint64_t wave_scan_max_u64(uint64_t v) {
  uint64_t w;
  w = dpp64<kDppRowShr1, 0xf>(0ull, v); v = w > v ? w : v;
  w = dpp64<kDppRowShr2, 0xf>(0ull, v); v = w > v ? w : v;
  w = dpp64<kDppRowShr4, 0xf>(0ull, v); v = w > v ? w : v;
  w = dpp64<kDppRowShr8, 0xf>(0ull, v); v = w > v ? w : v;
  w = dpp64<kDppRowBcast15, 0xa>(0ull, v); v = w > v ? w : v;
  w = dpp64<kDppRowBcast31, 0xc>(0ull, v); v = w > v ? w : v;
  return v;
}

__device__ __forceinline__ float wave_scan_max_f32(float v) {
  constexpr uint32_t kNegInf = 0xff800000u;
  v = nmax(v, __uint_as_float(dpp32<kDppRowShr1, 0xf>(kNegInf, __float_as_uint(v))));
  v = nmax(v, __uint_as_float(dpp32<kDppRowShr2, 0xf>(kNegInf, __float_as_uint(v))));
  v = nmax(v, __uint_as_float(dpp32<kDppRowShr4, 0xf>(kNegInf, __float_as_uint(v))));
  v = nmax(v, __uint_as_float(dpp32<kDppRowShr8, 0xf>(kNegInf, __float_as_uint(v))));
  v = nmax(v, __uint_as_float(dpp32<kDppRowBcast15, 0xa>(kNegInf, __float_as_uint(v))));
  v = nmax(v, __uint_as_float(dpp32<kDppRowBcast31, 0xc>(kNegInf, __float_as_uint(v))));
  return v;
}

__device__ __forceinline__ uint32_t lane_bcast_u32(uint32_t v, int lane) {
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), lane));
}
__device__ __forceinline__ uint64_t lane_bcast_u64(uint64_t v, int lane) {
  return (static_cast<uint64_t>(lane_bcast_u32(static_cast<uint32_t>(v >> 32), lane)) << 32) |
         lane_bcast_u32(static_cast<uint32_t>(v), lane);
}

// Reductions, result on every lane.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) { return lane_bcast_u64(wave_scan_max_u64(v), kWave - 1); }
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) { return lane_bcast_u64(wave_scan_add_u64(v), kWave - 1); }
__device__ __forceinline__ float wave_max_f32(float v) {
  return __uint_as_float(lane_bcast_u32(__float_as_uint(wave_scan_max_f32(v)), kWave - 1));
}

// Block-wide reductions; `smem` needs BLOCK/64 slots. Result broadcast to all.
// block_max_u64 writes its slots without a barrier first: no other use of
// `smem` may be in flight when it is called (one call per kernel, or a
// barrier between calls).
template <int BLOCK>
__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t* smem) {
  constexpr int kWaves = BLOCK / kWave;
  v = wave_max_u64(v);
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  if (lane == 0) smem[wid] = v;
  __syncthreads();
  uint64_t r = smem[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) r = smem[i] > r ? smem[i] : r;
  return r;
}

template <int BLOCK>
__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, uint64_t* smem) {
  constexpr int kWaves = BLOCK / kWave;
  v = wave_sum_u64(v);
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) smem[wid] = v;
  __syncthreads();
  uint64_t r = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) r += smem[i];
  return r;
}

template <int BLOCK>
__device__ __forceinline__ float block_max_f32(float v, float* smem) {
  constexpr int kWaves = BLOCK / kWave;
  v = wave_max_f32(v);
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) smem[wid] = v;
  __syncthreads();
  float r = smem[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) r = nmax(r, smem[i]);
  return r;
}

// ---------------------------------------------------------------------------
// Agent-scope atomics for the fused cross-workgroup epilogue.
//
// Cross-workgroup data in the fused epilogues travels ONLY through returning
// atomic read-modify-writes on agent scope: a producer publishes with an RMW,
// waits for that RMW to return (so it has been performed at the device
// coherence point), and only then arrives on the group counter with another
// RMW; the last arriver reads (and resets) the published words with RMWs.
// This avoids release/acquire fences, which on gfx950 write back and
// invalidate the L2 of the executing XCD on every workgroup.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t atomic_max_u64(uint64_t* p, uint64_t v) {
  return __hip_atomic_fetch_max(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t atomic_exchange_u64(uint64_t* p, uint64_t v) {
  return __hip_atomic_exchange(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t atomic_add_u64(uint64_t* p, uint64_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Force the value of a returning atomic to be available (s_waitcnt on its
// return) before any later memory operation is issued.
__device__ __forceinline__ void await_value(uint64_t v) {
  const uint32_t lo = static_cast<uint32_t>(v), hi = static_cast<uint32_t>(v >> 32);
  asm volatile("" ::"v"(lo), "v"(hi) : "memory");
}
__device__ __forceinline__ void await_value32(uint32_t v) { asm volatile("" ::"v"(v) : "memory"); }
// Arrive on a group counter after this thread's published RMWs have returned.
__device__ __forceinline__ uint32_t atomic_arrive(uint32_t* p) {
  return __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t atomic_add_u32(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t atomic_or_u32(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_or(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t atomic_exchange_u32(uint32_t* p, uint32_t v) {
  return __hip_atomic_exchange(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Device-coherent (agent-scope, relaxed) plain stores and loads: emitted as
// sc1 global memory operations that write through / bypass the per-XCD L2, so
// values published by one workgroup are visible to a workgroup on another XCD
// once the writer has drained its stores and signalled through an atomic.
__device__ __forceinline__ void store_sc(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_sc64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t load_sc(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_sc64(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until every store of this lane has been acknowledged by the device
// coherence point (vmcnt also counts stores on gfx9), and keep the compiler
// from moving memory operations across.
__device__ __forceinline__ void drain_stores() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0) expcnt(7) lgkmcnt(15)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ uint64_t atomic_load_u64(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void atomic_store_u64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void atomic_store_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace ls
