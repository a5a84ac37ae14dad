// Softmax statistics of logits rows: the lm_head epilogue of the draft's
// denoise step and of the target's verify pass.
//
// Replaces the torch sequence after the lm_head in the reference's denoise
// body, speculative_decoding/cache_aware.py:916-938
//   probs = softmax(logits.float()); pred = probs.argmax(-1);
//   conf = probs.gather(pred); masked_conf = where(cur == MASK, conf, -inf);
//   top = masked_conf.topk(n); cur.scatter_(top, pred[top]);
//   step_map.scatter_(top, step); per_pos_probs.index_copy_(top, probs[top])
// and the verify pass's target_probs = softmax(mask_logits.float())
// (cache_aware.py:1197-1198).
//
// Three launches, none of them larger than the logits:
//   row_partial_kernel   grid (P, M): each workgroup folds a slice of one row
//                        into (max, sum of exp(l - max), first index of max);
//   row_finalize_kernel  one workgroup: merges the P slices of every row in
//                        slice order, writes ids / conf, and (denoise) picks
//                        the rows to unmask;
//   row_probs_kernel     grid (P, M): probs = exp(l - max) / sum, for every
//                        row or only for the rows just unmasked.
// Every merge runs in a fixed order, so results are bit-reproducible.
#include <stdint.h>

#include "simsd_common.hpp"
#include "simsd_kernels.h"

namespace simsd {
namespace {

constexpr int kRowThreads = 256;
constexpr int64_t kNoIndex = INT64_MAX;
constexpr int kFinalizeWaves = 16;
constexpr int kMaxSelectRows = 64;    // the unmasking choice runs in one wave
constexpr int kBatch = 8;             // logits a thread loads at once

// Softmax state of a set of logits: the largest value, the sum of exp(l - mx)
// over the set, and the lowest index holding the largest value.
struct RowStat {
  float mx;
  float sm;
  int64_t ix;
};
static_assert(sizeof(RowStat) == 16, "workspace layout");

SIMSD_DEV RowStat stat_empty() { return RowStat{-INFINITY, 0.f, kNoIndex}; }

// Fold element e (value l) into s; elements arrive in increasing e.
SIMSD_DEV void stat_push(RowStat& s, float l, int64_t e) {
  if (l > s.mx) {
    s.sm = s.sm * expf(s.mx - l) + 1.f;
    s.mx = l;
    s.ix = e;
  } else if (l == s.mx) {
    if (l != -INFINITY) s.sm += 1.f;
    if (e < s.ix) s.ix = e;
  } else {
    s.sm += expf(l - s.mx);
  }
}

// Commutative merge of two states (bitwise: merge(a, b) == merge(b, a)).
SIMSD_DEV RowStat stat_merge(const RowStat& a, const RowStat& b) {
  RowStat r;
  r.mx = fmaxf(a.mx, b.mx);
  if (a.mx > b.mx) r.ix = a.ix;
  else if (b.mx > a.mx) r.ix = b.ix;
  else r.ix = a.ix < b.ix ? a.ix : b.ix;
  if (r.mx == -INFINITY) r.sm = 0.f;
  else r.sm = a.sm * expf(a.mx - r.mx) + b.sm * expf(b.mx - r.mx);
  return r;
}

SIMSD_DEV RowStat stat_shfl_xor(const RowStat& s, int d) {
  RowStat o;
  o.mx = __shfl_xor(s.mx, d);
  o.sm = __shfl_xor(s.sm, d);
  const int lo = __shfl_xor((int)(uint32_t)s.ix, d);
  const int hi = __shfl_xor((int)(uint32_t)((uint64_t)s.ix >> 32), d);
  o.ix = (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
  return o;
}

// Butterfly over the wave; every lane ends with the same state.
SIMSD_DEV RowStat stat_wave(RowStat s) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) s = stat_merge(s, stat_shfl_xor(s, d));
  return s;
}

template <int DT>
__global__ __launch_bounds__(kRowThreads) void row_partial_kernel(const char* __restrict__ logits, int64_t slm,
                                                                  int64_t V, int64_t chunk,
                                                                  RowStat* __restrict__ part) {
  __shared__ RowStat wres[kRowThreads / 64];
  const int64_t m = blockIdx.y;
  const int P = gridDim.x;
  const int64_t e0 = (int64_t)blockIdx.x * chunk;
  const int64_t e1 = min(V, e0 + chunk);
  const char* row = logits + m * slm * DTypeInfo<DT>::kSize;
  RowStat s = stat_empty();
  // kBatch loads issued together, then folded in index order
  for (int64_t b = e0 + threadIdx.x; b < e1; b += kBatch * kRowThreads) {
    float v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t e = b + (int64_t)u * kRowThreads;
      v[u] = load_elem<DT>(row, e < e1 ? e : e1 - 1);   // unconditional (no wait at a branch join)
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t e = b + (int64_t)u * kRowThreads;
      if (e < e1) stat_push(s, v[u], e);
    }
  }
  s = stat_wave(s);
  if ((threadIdx.x & 63) == 0) wres[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    RowStat t = wres[0];
#pragma unroll
    for (int w = 1; w < kRowThreads / 64; ++w) t = stat_merge(t, wres[w]);
    part[m * P + blockIdx.x] = t;
  }
}

// Per row: merge the P slice states (lane l takes slices l, l + 64, ...),
// ids[m] = first index of the maximum, conf[m] = its softmax probability
// 1 / sum, rowstat[m] = (max, sum) for the probabilities pass.
// Unmasking (cur_ids != null, M <= 64): among rows with cur_ids == mask_id the
// n_unmask largest conf win (rows not masked count as -inf, so they are taken
// only when fewer than n_unmask rows are masked, as torch.topk would); equal
// values go to the lower row.  Winners get cur_ids[m] = ids[m],
// step_map[m] = step and sel[m] = 1.
__global__ __launch_bounds__(64 * kFinalizeWaves) void row_finalize_kernel(
    const RowStat* __restrict__ part, int P, int64_t M, int64_t* __restrict__ ids, float* __restrict__ conf,
    float2* __restrict__ rowstat, int64_t* cur_ids, int64_t mask_id, int n_unmask, int64_t* step_map,
    int64_t step, int32_t* sel) {
  __shared__ float sh_conf[kMaxSelectRows];
  __shared__ int64_t sh_ids[kMaxSelectRows];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  for (int64_t m = wv; m < M; m += kFinalizeWaves) {
    RowStat s = stat_empty();
    for (int p = lane; p < P; p += 64) s = stat_merge(s, part[m * P + p]);
    s = stat_wave(s);
    if (lane == 0) {
      const float c = s.sm > 0.f ? 1.f / s.sm : __builtin_nanf("");
      const int64_t id = s.ix == kNoIndex ? 0 : s.ix;
      ids[m] = id;
      conf[m] = c;
      rowstat[m] = make_float2(s.mx, s.sm);
      if (cur_ids != nullptr) {
        sh_conf[m] = c;
        sh_ids[m] = id;
      }
    }
  }
  if (cur_ids == nullptr) return;
  __syncthreads();
  if (wv != 0) return;
  const bool live = lane < M;
  const float key = live && cur_ids[lane] == mask_id ? sh_conf[lane] : -INFINITY;
  int rank = 0;
  for (int j = 0; j < (int)M; ++j) {
    const float kj = __shfl(key, j);
    rank += (kj > key || (kj == key && j < lane)) ? 1 : 0;
  }
  const bool win = live && rank < n_unmask;
  if (live) sel[lane] = win ? 1 : 0;
  if (win) {
    cur_ids[lane] = sh_ids[lane];
    if (step_map != nullptr) step_map[lane] = step;
  }
}

// probs[m, e] = exp(l - max) / sum for rows with sel[m] (every row when sel
// is null).
template <int DT>
__global__ __launch_bounds__(kRowThreads) void row_probs_kernel(const char* __restrict__ logits, int64_t slm,
                                                                int64_t V, int64_t chunk,
                                                                const float2* __restrict__ rowstat,
                                                                const int32_t* sel, float* __restrict__ probs,
                                                                int64_t spm) {
  const int64_t m = blockIdx.y;
  if (sel != nullptr && sel[m] == 0) return;
  const float2 st = rowstat[m];
  const int64_t e0 = (int64_t)blockIdx.x * chunk;
  const int64_t e1 = min(V, e0 + chunk);
  const char* row = logits + m * slm * DTypeInfo<DT>::kSize;
  float* out = probs + m * spm;
  for (int64_t b = e0 + threadIdx.x; b < e1; b += kBatch * kRowThreads) {
    float v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t e = b + (int64_t)u * kRowThreads;
      v[u] = load_elem<DT>(row, e < e1 ? e : e1 - 1);   // unconditional (no wait at a branch join)
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t e = b + (int64_t)u * kRowThreads;
      if (e < e1) out[e] = expf(v[u] - st.x) / st.y;
    }
  }
}

// Slices per row: about 2048 logits per workgroup, at most 1024 slices.
struct RowPlan {
  int P;
  int64_t chunk;
  int64_t part_off, stat_off, sel_off, bytes;
};

inline int64_t round_up(int64_t a, int64_t b) { return (a + b - 1) / b * b; }

RowPlan row_plan(int64_t M, int64_t V) {
  RowPlan p{};
  int64_t P = (V + 2047) / 2048;
  if (P > 1024) P = 1024;
  if (P < 1) P = 1;
  p.chunk = round_up((V + P - 1) / P, kRowThreads);
  p.P = (int)((V + p.chunk - 1) / p.chunk);
  if (p.P < 1) p.P = 1;
  p.part_off = 0;
  p.stat_off = round_up(M * p.P * (int64_t)sizeof(RowStat), 256);
  p.sel_off = p.stat_off + round_up(M * (int64_t)sizeof(float2), 256);
  p.bytes = p.sel_off + round_up(M * (int64_t)sizeof(int32_t), 256);
  return p;
}

int check_rows(const char* what, const void* logits, int64_t M, int64_t V, int dtype, const void* ws,
               int64_t ws_bytes, const RowPlan& pl) {
  if (dtype != kBF16 && dtype != kF16 && dtype != kF32) return set_error("%s: unsupported dtype code %d", what, dtype);
  if (M < 0 || V <= 0) return set_error("%s: bad sizes M=%lld V=%lld", what, (long long)M, (long long)V);
  if (M > 65535) return set_error("%s: M=%lld exceeds 65535 rows", what, (long long)M);
  if (logits == nullptr) return set_error("%s: null logits", what);
  if (ws == nullptr || ws_bytes < pl.bytes || (reinterpret_cast<uintptr_t>(ws) & 15u) != 0)
    return set_error("%s: needs a 16-byte aligned workspace of %lld bytes (got %lld)", what, (long long)pl.bytes,
                     (long long)ws_bytes);
  return 0;
}

template <int DT>
void launch_rows(const char* logits, int64_t slm, int64_t M, int64_t V, const RowPlan& pl, char* ws,
                 int64_t* ids, float* conf, int64_t* cur_ids, int64_t mask_id, int n_unmask, int64_t* step_map,
                 int64_t step, float* probs, int64_t spm, hipStream_t stream) {
  RowStat* part = reinterpret_cast<RowStat*>(ws + pl.part_off);
  float2* rowstat = reinterpret_cast<float2*>(ws + pl.stat_off);
  int32_t* sel = reinterpret_cast<int32_t*>(ws + pl.sel_off);
  const dim3 grid((unsigned)pl.P, (unsigned)M);
  hipLaunchKernelGGL(row_partial_kernel<DT>, grid, dim3(kRowThreads), 0, stream, logits, slm, V, pl.chunk, part);
  hipLaunchKernelGGL(row_finalize_kernel, dim3(1), dim3(64 * kFinalizeWaves), 0, stream, part, pl.P, M, ids, conf,
                     rowstat, cur_ids, mask_id, n_unmask, step_map, step, sel);
  if (probs != nullptr)
    hipLaunchKernelGGL(row_probs_kernel<DT>, grid, dim3(kRowThreads), 0, stream, logits, slm, V, pl.chunk, rowstat,
                       cur_ids != nullptr ? sel : nullptr, probs, spm);
}

void dispatch_rows(int dtype, const void* logits, int64_t slm, int64_t M, int64_t V, const RowPlan& pl, void* ws,
                   int64_t* ids, float* conf, int64_t* cur_ids, int64_t mask_id, int n_unmask, int64_t* step_map,
                   int64_t step, float* probs, int64_t spm, hipStream_t stream) {
  const char* l = static_cast<const char*>(logits);
  char* w = static_cast<char*>(ws);
  switch (dtype) {
    case kBF16:
      launch_rows<kBF16>(l, slm, M, V, pl, w, ids, conf, cur_ids, mask_id, n_unmask, step_map, step, probs, spm, stream);
      break;
    case kF16:
      launch_rows<kF16>(l, slm, M, V, pl, w, ids, conf, cur_ids, mask_id, n_unmask, step_map, step, probs, spm, stream);
      break;
    default:
      launch_rows<kF32>(l, slm, M, V, pl, w, ids, conf, cur_ids, mask_id, n_unmask, step_map, step, probs, spm, stream);
      break;
  }
}

}  // namespace
}  // namespace simsd

using namespace simsd;

extern "C" int64_t simsd_softmax_argmax_workspace_bytes(int64_t M, int64_t V) {
  if (M < 0 || V <= 0) return -1;
  return row_plan(M, V).bytes;
}

extern "C" int simsd_softmax_argmax(const void* logits, int64_t slm, int64_t M, int64_t V, int dtype, int64_t* ids,
                                    float* conf, float* probs, int64_t spm, void* workspace,
                                    int64_t workspace_bytes, void* stream) {
  const RowPlan pl = row_plan(M, V);
  if (check_rows("softmax_argmax", logits, M, V, dtype, workspace, workspace_bytes, pl) != 0) return -1;
  if (M == 0) return 0;
  if (ids == nullptr || conf == nullptr) return set_error("softmax_argmax: null ids or conf");
  dispatch_rows(dtype, logits, slm, M, V, pl, workspace, ids, conf, nullptr, 0, 0, nullptr, 0, probs, spm,
                static_cast<hipStream_t>(stream));
  return check_launch("softmax_argmax");
}

extern "C" int simsd_denoise_select(const void* logits, int64_t slm, int64_t M, int64_t V, int dtype,
                                    int64_t* cur_ids, int64_t mask_id, int n_unmask, int64_t* step_map, int64_t step,
                                    float* per_pos_probs, int64_t spp, int64_t* ids, float* conf, void* workspace,
                                    int64_t workspace_bytes, void* stream) {
  const RowPlan pl = row_plan(M, V);
  if (check_rows("denoise_select", logits, M, V, dtype, workspace, workspace_bytes, pl) != 0) return -1;
  if (M > kMaxSelectRows) return set_error("denoise_select: M=%lld exceeds %d rows", (long long)M, kMaxSelectRows);
  if (n_unmask < 0 || n_unmask > M)
    return set_error("denoise_select: n_unmask=%d outside [0, %lld]", n_unmask, (long long)M);
  if (M == 0) return 0;
  if (cur_ids == nullptr || ids == nullptr || conf == nullptr) return set_error("denoise_select: null pointer");
  dispatch_rows(dtype, logits, slm, M, V, pl, workspace, ids, conf, cur_ids, mask_id, n_unmask, step_map, step,
                per_pos_probs, spp, static_cast<hipStream_t>(stream));
  return check_launch("denoise_select");
}
