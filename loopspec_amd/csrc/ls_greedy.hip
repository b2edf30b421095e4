// (b) Greedy verification for gfx950.
//
// One launch covers every row of the step. Each workgroup owns one segment of
// one row, sized so that every lane issues about six 16-byte loads up front and
// several workgroups share a CU; a lane keeps a (group-max, vector) candidate,
// resolves the exact first index inside the winning vector, and the block
// reduces packed (value, -index) keys. Rows of one batch element meet in the
// fused epilogue: each workgroup publishes its key with an agent-scope
// atomicMax, waits for it to return, and arrives on the element's counter; the
// last arriver reads the keys back with atomic exchanges (which also re-zero
// the workspace) and runs the accept-prefix scan.
//
// Reference semantics: torch.argmax over the endpoint rows
// (sglang_recurrent/loopspec/decisions.py:116) and the final-endpoint rule
// (decisions.py:157-170) applied along the accept prefix (pipeline.py:365-412).
#include "ls_common.hpp"
#include "ls_runtime.hpp"

namespace ls {
namespace {

constexpr int kUnroll = 8;

struct GreedyParams {
  const char* target;        // row (b, i) at target + b*t_bstride + i*t_pstride (bytes)
  int64_t t_bstride, t_pstride;
  const char* draft;         // NULL when draft ids are supplied
  int64_t d_bstride, d_pstride;
  const int64_t* draft_tokens;
  int64_t vocab;
  int k;                     // draft positions (verify mode); 0 in argmax mode
  int rows_per_group;        // argmax: 1; verify: (k+1) [+ k when draft logits given]
  int splits;                // workgroups per row
  int direct;                // argmax mode with splits == 1: write out[] directly
  int64_t* out;              // argmax mode output [rows]
  int32_t* accept_len;       // verify outputs
  int64_t* tokens;
  int64_t* row_argmax;
  uint64_t* slots;           // workspace: one key per row
  uint32_t* counters;        // workspace: one arrival counter per group
};

// Row pointer of global row r (verify rows are grouped per batch element:
// target positions 0..k first, then draft positions 0..k-1).
__device__ __forceinline__ const char* row_ptr(const GreedyParams& p, int64_t r) {
  if (p.k == 0) return p.target + r * p.t_pstride;
  const int64_t b = r / p.rows_per_group;
  const int j = static_cast<int>(r - b * p.rows_per_group);
  if (j <= p.k) return p.target + b * p.t_bstride + j * p.t_pstride;
  return p.draft + b * p.d_bstride + (j - p.k - 1) * p.d_pstride;
}

// First-index argmax key of this lane's share of vectors [v0, v1) of a row.
// The lane's vectors are v0 + lane + j*BLOCK for j < n. Loads go through a
// clamped address (lanes past their last vector re-read it and ignore the
// result), so a batch of kUnroll loads is issued without branches and each
// vector is consumed as soon as its own load returns.
template <int DT, int BLOCK>
__device__ __forceinline__ uint64_t thread_argmax_vec(const u32x4* __restrict__ src, int64_t v0, int64_t v1) {
  constexpr int EPV = Elem<DT>::kPerVec;
  const int64_t first = v0 + threadIdx.x;
  if (first >= v1) return 0;
  const int n = static_cast<int>((v1 - first + BLOCK - 1) / BLOCK);
  const u32x4* __restrict__ p = src + first;
  float best = -__builtin_inff();
  int bestj = 0;
  u32x4 bestd = {0u, 0u, 0u, 0u};
  for (int j0 = 0; j0 < n; j0 += kUnroll) {
    u32x4 d[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int j = j0 + u < n ? j0 + u : n - 1;
      d[u] = __builtin_nontemporal_load(p + static_cast<int64_t>(j) * BLOCK);
    }
    // Seeding with the lane's first vector makes an all -inf share resolve to
    // its first element without a sentinel.
    if (j0 == 0) bestd = d[0];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const float g = vec_max<DT>(d[u]);
      // Vectors arrive in increasing index order, so a strict '>' keeps the
      // earliest vector holding the maximum; a NaN beats any number once.
      const bool take = (j0 + u < n) & ((g > best) | ((g != g) & (best == best)));
      best = take ? g : best;
      bestj = take ? j0 + u : bestj;
      bestd = take ? d[u] : bestd;
    }
  }
  const bool is_nan = best != best;
  int e = 0;
#pragma unroll
  for (int q = EPV - 1; q >= 0; --q) {
    const float x = vec_elem<DT>(bestd, q);
    if (is_nan ? (x != x) : (x == best)) e = q;
  }
  const int64_t v = first + static_cast<int64_t>(bestj) * BLOCK;
  return argmax_key(best, static_cast<uint32_t>(v * EPV + e));
}

// Unaligned fallback: element-wise loads.
template <int DT, int BLOCK>
__device__ __forceinline__ uint64_t thread_argmax_scalar(const char* row, int64_t i0, int64_t i1) {
  float best = 0.f;
  int64_t besti = -1;
  for (int64_t i = i0 + threadIdx.x; i < i1; i += BLOCK) {
    const float x = load_elem<DT>(row, i);
    const bool take = (besti < 0) | (x > best) | ((x != x) & (best == best));
    if (take) {
      best = x;
      besti = i;
    }
  }
  return besti < 0 ? 0 : argmax_key(best, static_cast<uint32_t>(besti));
}

// Runs on every lane of the last workgroup of group g (a block-uniform
// branch). Lane j reads row j's combined key with an exchange, which also
// leaves the slot zeroed, so all rows' reads are in flight together; lane 0
// then runs the scan.
template <int BLOCK>
__device__ void finalize_group(const GreedyParams& p, int64_t g, int64_t* ids) {
  uint64_t* slots = p.slots + g * p.rows_per_group;
  const int lane = threadIdx.x;
  for (int j = lane; j < p.rows_per_group; j += BLOCK) ids[j] = argmax_key_index(atomic_exchange_u64(slots + j, 0));
  if (lane == 0) atomic_exchange_u32(p.counters + g, 0u);
  __syncthreads();
  if (lane != 0) return;
  if (p.k == 0) {
    p.out[g] = ids[0];
    return;
  }
  const int k = p.k;
  int accepted = 0;
  bool run = true;
  for (int i = 0; i <= k; ++i) {
    const int64_t t = ids[i];
    const int64_t d = i < k ? (p.draft ? ids[k + 1 + i] : p.draft_tokens[g * k + i]) : -1;
    p.tokens[g * (k + 1) + i] = run ? t : -1;
    if (run && i < k && d == t) {
      ++accepted;
    } else {
      run = false;
    }
    if (p.row_argmax) {
      p.row_argmax[g * (2 * k + 1) + i] = t;
      if (i < k) p.row_argmax[g * (2 * k + 1) + k + 1 + i] = d;
    }
  }
  p.accept_len[g] = accepted;
}

template <int DT, bool VEC, int BLOCK>
__global__ __launch_bounds__(BLOCK) void greedy_kernel(GreedyParams p) {
  __shared__ uint64_t red[BLOCK / kWave];
  __shared__ int64_t ids[2 * 64 + 1];
  __shared__ int last;
  const int64_t r = blockIdx.x / p.splits;
  const int split = static_cast<int>(blockIdx.x - r * p.splits);
  const char* row = row_ptr(p, r);

  uint64_t key;
  if constexpr (VEC) {
    constexpr int EPV = Elem<DT>::kPerVec;
    const int64_t nvec = p.vocab / EPV;
    const int64_t per = (nvec + p.splits - 1) / p.splits;
    const int64_t v0 = split * per;
    const int64_t v1 = v0 + per < nvec ? v0 + per : nvec;
    key = thread_argmax_vec<DT, BLOCK>(reinterpret_cast<const u32x4*>(row), v0, v1);
  } else {
    const int64_t per = (p.vocab + p.splits - 1) / p.splits;
    const int64_t i0 = split * per;
    const int64_t i1 = i0 + per < p.vocab ? i0 + per : p.vocab;
    key = thread_argmax_scalar<DT, BLOCK>(row, i0, i1);
  }
  key = block_max_u64<BLOCK>(key, red);

  if (p.direct) {
    if (threadIdx.x == 0) p.out[r] = argmax_key_index(key);
    return;
  }
  const int64_t g = r / p.rows_per_group;
  if (threadIdx.x == 0) {
    await_value(atomic_max_u64(p.slots + r, key));
    const uint32_t prev = atomic_arrive(p.counters + g);
    last = prev == static_cast<uint32_t>(p.rows_per_group * p.splits - 1);
  }
  __syncthreads();
  if (last) finalize_group<BLOCK>(p, g, ids);
}

uint64_t workspace_bytes(int64_t rows, int64_t groups) {
  const uint64_t slots = static_cast<uint64_t>(rows) * 8u;
  const uint64_t counters = (static_cast<uint64_t>(groups) * 4u + 7u) & ~7ull;
  return (slots + counters + 255u) & ~255ull;
}

struct Shape {
  int block;
  int splits;
};

// Workgroup shape. Measured on MI355X (C2: 320 bf16 rows of 49152): 256-lane
// workgroups, one per row, each lane streaming 24 vectors in batches of
// kUnroll, beat both larger workgroups and split rows -- splitting adds
// same-address atomics to the epilogue. Rows are split only when there are
// fewer rows than CUs, keeping at least one full batch of loads per lane.
Shape choose_shape(int64_t rows, int64_t vocab, int elem_bytes) {
  const int64_t nvec = vocab * elem_bytes / 16 > 0 ? vocab * elem_bytes / 16 : 1;
  int64_t block = option("greedy_block");
  if (block != 256 && block != 512 && block != 1024) block = 256;
  int64_t s = option("greedy_splits");
  if (s <= 0) {
    const int64_t cus = static_cast<int64_t>(device_cu_count());
    s = rows >= cus ? 1 : (cus + rows - 1) / rows;
    const int64_t by_loads = nvec / (block * kUnroll);
    if (s > by_loads) s = by_loads;
  }
  const int64_t max_s = nvec / (block * 2) > 0 ? nvec / (block * 2) : 1;
  if (s > max_s) s = max_s;
  if (s < 1) s = 1;
  if (s > 64) s = 64;
  return Shape{static_cast<int>(block), static_cast<int>(s)};
}

template <int DT, int BLOCK>
void launch_block(const GreedyParams& p, int64_t total_rows, bool vec, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(total_rows * p.splits));
  if (vec) {
    hipLaunchKernelGGL((greedy_kernel<DT, true, BLOCK>), grid, dim3(BLOCK), 0, st, p);
  } else {
    hipLaunchKernelGGL((greedy_kernel<DT, false, BLOCK>), grid, dim3(BLOCK), 0, st, p);
  }
}

template <int DT>
void launch_dt(const GreedyParams& p, int block, int64_t total_rows, bool vec, hipStream_t st) {
  if (block == 1024) {
    launch_block<DT, 1024>(p, total_rows, vec, st);
  } else if (block == 512) {
    launch_block<DT, 512>(p, total_rows, vec, st);
  } else {
    launch_block<DT, 256>(p, total_rows, vec, st);
  }
}

int launch(const GreedyParams& p, int dtype, int block, int64_t total_rows, bool vec, hipStream_t st) {
  switch (dtype) {
    case LS_DTYPE_F32: launch_dt<F32>(p, block, total_rows, vec, st); break;
    case LS_DTYPE_BF16: launch_dt<BF16>(p, block, total_rows, vec, st); break;
    case LS_DTYPE_F16: launch_dt<F16>(p, block, total_rows, vec, st); break;
    default: return fail(LS_ERR_VALUE, "unsupported logits dtype");
  }
  return check_launch("greedy kernel launch");
}

}  // namespace
}  // namespace ls

using namespace ls;

extern "C" {

uint64_t ls_argmax_rows_workspace(int64_t rows, int64_t vocab) {
  (void)vocab;
  return rows > 0 ? workspace_bytes(rows, rows) : 0;
}

int ls_argmax_rows(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t row_stride,
                   int64_t* out, void* workspace, uint64_t ws_bytes, ls_stream_t stream) {
  const int eb = dtype_bytes(dtype);
  if (eb == 0) return fail(LS_ERR_VALUE, "unsupported logits dtype");
  if (rows < 0 || vocab <= 0 || vocab > 0x7fffffffLL) return fail(LS_ERR_VALUE, "argmax: invalid rows/vocab");
  if (rows == 0) return LS_OK;
  if (logits == nullptr || out == nullptr) return fail(LS_ERR_VALUE, "argmax: NULL pointer");
  if (rows > 0x7fffffffLL / 64) return fail(LS_ERR_VALUE, "argmax: too many rows");
  GreedyParams p{};
  p.target = static_cast<const char*>(logits);
  p.t_pstride = row_stride * eb;
  p.vocab = vocab;
  p.k = 0;
  p.rows_per_group = 1;
  const Shape shape = choose_shape(rows, vocab, eb);
  p.splits = shape.splits;
  p.out = out;
  if (p.splits > 1) {
    if (workspace == nullptr || ws_bytes < workspace_bytes(rows, rows)) {
      // Without scratch fall back to one workgroup per row.
      p.splits = 1;
    } else {
      p.slots = static_cast<uint64_t*>(workspace);
      p.counters = reinterpret_cast<uint32_t*>(p.slots + rows);
    }
  }
  p.direct = p.splits == 1;
  const bool vec = aligned16(logits) && ((row_stride * eb) % 16 == 0) && ((vocab * eb) % 16 == 0);
  return launch(p, dtype, shape.block, rows, vec, static_cast<hipStream_t>(stream));
}

uint64_t ls_greedy_verify_workspace(int64_t batch, int64_t k, int64_t vocab) {
  (void)vocab;
  if (batch <= 0 || k < 0) return 0;
  return workspace_bytes(batch * (2 * k + 1), batch);
}

int ls_greedy_verify(const void* target_logits, int64_t target_batch_stride, int64_t target_pos_stride,
                     const void* draft_logits, int64_t draft_batch_stride, int64_t draft_pos_stride,
                     const int64_t* draft_tokens, int dtype, int64_t batch, int64_t k, int64_t vocab,
                     int32_t* accept_len, int64_t* tokens, int64_t* row_argmax, void* workspace,
                     uint64_t ws_bytes, ls_stream_t stream) {
  const int eb = dtype_bytes(dtype);
  if (eb == 0) return fail(LS_ERR_VALUE, "unsupported logits dtype");
  if (batch < 0 || k < 1 || k > 64 || vocab <= 0 || vocab > 0x7fffffffLL)
    return fail(LS_ERR_VALUE, "greedy_verify: invalid batch/k/vocab (need 1 <= k <= 64)");
  if (batch == 0) return LS_OK;
  if (target_logits == nullptr || accept_len == nullptr || tokens == nullptr)
    return fail(LS_ERR_VALUE, "greedy_verify: NULL pointer");
  if (draft_logits == nullptr && draft_tokens == nullptr)
    return fail(LS_ERR_VALUE, "greedy_verify: need draft logits or draft tokens");
  const int rpg = static_cast<int>(draft_logits ? 2 * k + 1 : k + 1);
  const int64_t total = batch * rpg;
  if (total > 0x7fffffffLL / 64) return fail(LS_ERR_VALUE, "greedy_verify: too many rows");
  if (workspace == nullptr || ws_bytes < workspace_bytes(total, batch))
    return fail(LS_ERR_VALUE, "greedy_verify: workspace too small");
  GreedyParams p{};
  p.target = static_cast<const char*>(target_logits);
  p.t_bstride = target_batch_stride * eb;
  p.t_pstride = target_pos_stride * eb;
  p.draft = static_cast<const char*>(draft_logits);
  p.d_bstride = draft_batch_stride * eb;
  p.d_pstride = draft_pos_stride * eb;
  p.draft_tokens = draft_tokens;
  p.vocab = vocab;
  p.k = static_cast<int>(k);
  p.rows_per_group = rpg;
  const Shape shape = choose_shape(total, vocab, eb);
  p.splits = shape.splits;
  p.direct = 0;
  p.accept_len = accept_len;
  p.tokens = tokens;
  p.row_argmax = row_argmax;
  p.slots = static_cast<uint64_t*>(workspace);
  p.counters = reinterpret_cast<uint32_t*>(p.slots + total);
  bool vec = aligned16(target_logits) && (p.t_bstride % 16 == 0) && (p.t_pstride % 16 == 0) &&
             ((vocab * eb) % 16 == 0);
  if (draft_logits)
    vec = vec && aligned16(draft_logits) && (p.d_bstride % 16 == 0) && (p.d_pstride % 16 == 0);
  return launch(p, dtype, shape.block, total, vec, static_cast<hipStream_t>(stream));
}

}  // extern "C"
