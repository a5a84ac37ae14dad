// Skinny GEMM y[M,N] = x[M,K] . w[N,K]^T (+ bias) for gfx950.
//
// Replaces the Triton _thin_gemv_kernel / _thin_gemv_reduce pair of
// kernels/thin_linear_fused.py:67-171 (reference).  Design for MI355X:
//   * the weight streams straight from HBM into MFMA A operands with 128-bit
//     non-temporal loads (16 rows x 64 B per wave per k-step), double-buffered;
//   * the few activation rows are the MFMA B operand (16 columns per block,
//     masked lanes for M < 16), read through L1/L2 where they stay resident;
//   * a workgroup owns RB*16 weight rows and splits K across KS waves, whose
//     fp32 partials meet in LDS in fixed wave order;
//   * optional split-K across workgroups (SPLIT) for narrow N: every workgroup
//     writes an fp32 partial tile, and the last one to arrive (device-scope
//     counter) sums the SPLIT partials in index order -- deterministic, one
//     launch, no atomics on data, and it leaves its counter at zero again.
#include <stdarg.h>
#include <stdio.h>

#include "simsd_common.hpp"
#include "simsd_kernels.h"

namespace simsd {

struct ThinArgs {
  const char* x;
  int64_t sxm, sxk;          // element strides
  const char* w;
  int64_t swn, swk;
  const char* bias;          // nullable, element stride sb
  int64_t sb;
  char* y;
  int64_t sym, syn;
  float* part;               // [split][M][N] fp32, used when split > 1
  uint32_t* counters;        // [gridDim.z][gridDim.x], zero between launches
  int64_t M, N, K;
  int steps;                 // ceil(K * esize / 64)
  int split;                 // workgroups along K
  int steps_per_split;
};

template <int DT, int RB, int CB, int KS, int U, bool FAST>
__global__ __launch_bounds__(64 * KS) void thin_gemm_kernel(ThinArgs a) {
  constexpr int ES = DTypeInfo<DT>::kSize;
  constexpr int NF = RB * CB;
  const int lane = threadIdx.x & 63;
  const int wk = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int64_t n_tile = (int64_t)blockIdx.x * (RB * 16);
  const int64_t m_tile = (int64_t)blockIdx.z * (CB * 16);
  const int split_id = blockIdx.y;

  // k-steps of this workgroup, then of this wave
  const int s_lo = split_id * a.steps_per_split;
  const int s_hi = min(a.steps, s_lo + a.steps_per_split);
  const int span = max(0, s_hi - s_lo);
  const int per_w = (span + KS - 1) / KS;
  const int w0 = s_lo + wk * per_w;
  const int w1 = min(s_hi, w0 + per_w);

  f32x4_t acc[RB][CB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const char* arow[RB];
  const char* brow[CB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int64_t n = min(n_tile + rb * 16 + r, a.N - 1);
    arow[rb] = a.w + n * a.swn * ES;
  }
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const int64_t m = m_tile + cb * 16 + r;
    brow[cb] = m < a.M ? a.x + m * a.sxm * ES : nullptr;
  }
  if (FAST) {
    accum_fast<DT, RB, CB, U>(arow, brow, w0, w1, g * kLaneBytes, a.K * ES, acc);
  } else {
    accum_generic<DT, RB, CB>(arow, a.swk * ES, brow, a.sxk * ES, w0, w1, g, a.K, acc);
  }

  __shared__ float red[KS > 1 ? (KS - 1) * NF * 4 * 64 : 1];
  reduce_waves<KS, NF>(reinterpret_cast<f32x4_t(&)[NF]>(acc), wk, lane, red);

  const bool single = a.split == 1;
  if (wk == 0) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int64_t m = m_tile + cb * 16 + r;
        const int64_t nb = n_tile + rb * 16 + 4 * g;
        if (m < a.M) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int64_t n = nb + j;
            if (n < a.N) {
              float v = acc[rb][cb][j];
              if (single) {
                if (a.bias != nullptr) v += load_elem<DT>(a.bias, n * a.sb);
                store_elem<DT>(a.y, m * a.sym + n * a.syn, v);
              } else {
                a.part[((int64_t)split_id * a.M + m) * a.N + n] = v;
              }
            }
          }
        }
      }
  }
  if (single) return;

  // ---- split-K: the last workgroup of this tile sums the partials in order
  __shared__ uint32_t s_last;
  __threadfence();
  __syncthreads();
  const int64_t cidx = (int64_t)blockIdx.z * gridDim.x + blockIdx.x;
  if (threadIdx.x == 0) {
    const uint32_t old = atomicAdd(&a.counters[cidx], 1u);
    s_last = (old == (uint32_t)(a.split - 1)) ? 1u : 0u;
  }
  __syncthreads();
  if (s_last == 0u) return;
  __threadfence();
  constexpr int TR = RB * 16, TC = CB * 16;
  for (int e = threadIdx.x; e < TR * TC; e += blockDim.x) {
    const int64_t n = n_tile + (e % TR);
    const int64_t m = m_tile + (e / TR);
    if (n < a.N && m < a.M) {
      float v = 0.f;
      for (int s = 0; s < a.split; ++s) v += a.part[((int64_t)s * a.M + m) * a.N + n];
      if (a.bias != nullptr) v += load_elem<DT>(a.bias, n * a.sb);
      store_elem<DT>(a.y, m * a.sym + n * a.syn, v);
    }
  }
  if (threadIdx.x == 0) a.counters[cidx] = 0u;
}

// ------------------------------------------------------------------ host side
namespace {

struct ThinPlan {
  int rb, cb, ks, split;
  bool fast;
  int64_t tiles_n, tiles_m;
  int steps, steps_per_split;
  int64_t counter_bytes, part_bytes;
};

inline int esize_of(int dtype) { return dtype == kF32 ? 4 : 2; }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr int kTargetWorkgroups = 512;   // 2 per CU on 256 CUs
constexpr int kMaxSplit = 16;

// Geometry only (no pointers): rows per workgroup, column blocks, waves per
// workgroup, split along K, and the workspace that split needs.
int plan_geometry(ThinPlan& pl, int64_t M, int64_t N, int64_t K, int dtype, int rb, int ks,
                  int split_k) {
  const int es = esize_of(dtype);
  pl.cb = M <= 16 ? 1 : 2;
  pl.rb = rb;
  pl.ks = ks;
  pl.tiles_n = (N + 16 * pl.rb - 1) / (16 * pl.rb);
  pl.tiles_m = (M + 16 * pl.cb - 1) / (16 * pl.cb);
  pl.steps = (int)((K * es + kStepBytes - 1) / kStepBytes);
  int split = split_k;
  if (split <= 0) {
    // Enough workgroups to put two on every CU, but never fewer than four
    // k-steps per wave.
    const int64_t wgs = pl.tiles_n * pl.tiles_m;
    split = (int)((kTargetWorkgroups + wgs - 1) / wgs);
    const int max_by_k = pl.steps / (pl.ks * 4);
    split = max(1, min(split, min(kMaxSplit, max_by_k)));
  }
  if (split > 1024) return set_error("thin_linear: split_k=%d exceeds 1024", split);
  pl.split = split;
  pl.steps_per_split = (pl.steps + split - 1) / split;
  pl.counter_bytes = split > 1 ? ((pl.tiles_n * pl.tiles_m * 4 + 255) / 256) * 256 : 0;
  pl.part_bytes = split > 1 ? (int64_t)split * M * N * 4 : 0;
  return 0;
}

inline int rb_of(int block_n) { return block_n >= 32 ? 2 : 1; }
inline int ks_of(int num_waves) {
  return num_waves <= 0 ? 4 : (num_waves <= 2 ? 2 : (num_waves <= 4 ? 4 : 8));
}

int make_plan(ThinPlan& pl, const void* x, int64_t sxm, int64_t sxk, const void* w, int64_t swn,
              int64_t swk, int64_t M, int64_t N, int64_t K, int dtype, int block_n, int split_k,
              int num_waves) {
  const int es = esize_of(dtype);
  const bool w_vec = swk == 1 && aligned16(w) && ((swn * es) % 16 == 0 || N == 1) && (K * es) % 16 == 0;
  const bool x_vec = sxk == 1 && aligned16(x) && ((sxm * es) % 16 == 0 || M == 1);
  const bool fast = w_vec && x_vec;
  // The strided path has a single shape: 16 rows per workgroup, 4 waves.
  if (plan_geometry(pl, M, N, K, dtype, fast ? rb_of(block_n) : 1, fast ? ks_of(num_waves) : 4,
                    split_k) != 0)
    return -1;
  pl.fast = fast;
  return 0;
}

template <int DT, int RB, int CB, int KS, bool FAST>
void launch_thin(const ThinPlan& pl, const ThinArgs& args, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  constexpr int U = (RB * CB == 1) ? 8 : 4;
  dim3 grid((unsigned)pl.tiles_n, (unsigned)pl.split, (unsigned)pl.tiles_m);
  hipLaunchKernelGGL((thin_gemm_kernel<DT, RB, CB, KS, U, FAST>), grid, dim3(64 * KS), 0, stream,
                     args);
}

template <int DT, int RB, int CB>
void dispatch_ks(const ThinPlan& pl, const ThinArgs& args, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  switch (pl.ks) {
    case 2: launch_thin<DT, RB, CB, 2, true>(pl, args, stream); break;
    case 8: launch_thin<DT, RB, CB, 8, true>(pl, args, stream); break;
    default: launch_thin<DT, RB, CB, 4, true>(pl, args, stream); break;
  }
}

template <int DT>
void dispatch_dt(const ThinPlan& pl, const ThinArgs& args, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (!pl.fast) {
    if (pl.cb == 1) launch_thin<DT, 1, 1, 4, false>(pl, args, stream);
    else launch_thin<DT, 1, 2, 4, false>(pl, args, stream);
    return;
  }
  if (pl.rb == 1 && pl.cb == 1) dispatch_ks<DT, 1, 1>(pl, args, stream);
  else if (pl.rb == 1) dispatch_ks<DT, 1, 2>(pl, args, stream);
  else if (pl.cb == 1) dispatch_ks<DT, 2, 1>(pl, args, stream);
  else dispatch_ks<DT, 2, 2>(pl, args, stream);
}

}  // namespace
}  // namespace simsd

using namespace simsd;

extern "C" int64_t simsd_thin_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int dtype,
                                                     int block_n, int split_k, int num_waves) {
  // Enough for either path: the requested geometry (vector-capable operands)
  // and the strided fallback (16 rows, 4 waves).
  ThinPlan a{}, b{};
  if (plan_geometry(a, M, N, K, dtype, rb_of(block_n), ks_of(num_waves), split_k) != 0) return -1;
  if (plan_geometry(b, M, N, K, dtype, 1, 4, split_k) != 0) return -1;
  const int64_t na = a.counter_bytes + a.part_bytes, nb = b.counter_bytes + b.part_bytes;
  return na > nb ? na : nb;
}

extern "C" int simsd_thin_linear(const void* x, int64_t sxm, int64_t sxk, const void* w,
                                 int64_t swn, int64_t swk, const void* bias, int64_t sb, void* y,
                                 int64_t sym, int64_t syn, int64_t M, int64_t N, int64_t K,
                                 int dtype, int block_n, int split_k, int num_waves,
                                 void* workspace, int64_t workspace_bytes, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (dtype != kBF16 && dtype != kF16 && dtype != kF32)
    return set_error("thin_linear: unsupported dtype code %d", dtype);
  if (M < 0 || N < 0 || K < 0) return set_error("thin_linear: negative size");
  if (M == 0 || N == 0) return 0;
  if (K == 0) return set_error("thin_linear: K == 0 must be handled by the caller");
  if (x == nullptr || w == nullptr || y == nullptr) return set_error("thin_linear: null pointer");
  if (K * (int64_t)esize_of(dtype) > ((int64_t)1 << 31) - 64)
    return set_error("thin_linear: K=%lld too large", (long long)K);
  ThinPlan pl{};
  if (make_plan(pl, x, sxm, sxk, w, swn, swk, M, N, K, dtype, block_n, split_k, num_waves) != 0)
    return -1;
  if (pl.tiles_n > 0x7fffffff || pl.tiles_m > 65535)
    return set_error("thin_linear: grid too large (N=%lld, M=%lld)", (long long)N, (long long)M);
  ThinArgs args{};
  args.x = static_cast<const char*>(x);
  args.sxm = sxm; args.sxk = sxk;
  args.w = static_cast<const char*>(w);
  args.swn = swn; args.swk = swk;
  args.bias = static_cast<const char*>(bias);
  args.sb = sb;
  args.y = static_cast<char*>(y);
  args.sym = sym; args.syn = syn;
  args.M = M; args.N = N; args.K = K;
  args.steps = pl.steps;
  args.split = pl.split;
  args.steps_per_split = pl.steps_per_split;
  if (pl.split > 1) {
    const int64_t need = pl.counter_bytes + pl.part_bytes;
    if (workspace == nullptr || workspace_bytes < need)
      return set_error("thin_linear: split_k=%d needs a %lld-byte workspace (got %lld)", pl.split,
                       (long long)need, (long long)workspace_bytes);
    if (!aligned16(workspace)) return set_error("thin_linear: workspace must be 16-byte aligned");
    args.counters = static_cast<uint32_t*>(workspace);
    args.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + pl.counter_bytes);
  }
  switch (dtype) {
    case kBF16: dispatch_dt<kBF16>(pl, args, stream); break;
    case kF16: dispatch_dt<kF16>(pl, args, stream); break;
    default: dispatch_dt<kF32>(pl, args, stream); break;
  }
  return check_launch("thin_linear");
}

extern "C" int simsd_thin_linear_plan(int64_t M, int64_t N, int64_t K, int dtype, int block_n,
                                      int split_k, int num_waves, int* out4) {
  // (rows per workgroup, columns per block, waves per workgroup, split) of the
  // vector-path geometry; lets the Python side report the config it runs.
  ThinPlan pl{};
  if (plan_geometry(pl, M, N, K, dtype, rb_of(block_n), ks_of(num_waves), split_k) != 0) return -1;
  out4[0] = 16 * pl.rb;
  out4[1] = 16 * pl.cb;
  out4[2] = pl.ks;
  out4[3] = pl.split;
  return 0;
}
