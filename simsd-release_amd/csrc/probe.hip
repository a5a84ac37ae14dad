// Measurement probes (no reference counterpart): the floors the skinny linear
// is measured against, and the VALU form of the M <= 4 linear it is compared
// with.
//   * an empty launch: what a kernel boundary costs inside a HIP graph;
//   * a pure read of a weight matrix in thin_gemv4_kernel's access pattern --
//     rows_per_wg weight rows per workgroup, `waves` waves splitting each row,
//     every load instruction 4 rows x 256 contiguous bytes, non-temporal --
//     with no arithmetic but an XOR fold (one 4-byte store per workgroup keeps
//     the loads live).  Its time is the floor a GEMV over the same bytes and
//     grid can reach.
#include "simsd_common.hpp"
#include "simsd_kernels.h"

namespace simsd {
namespace {

constexpr int kProbeBatch = 8;   // load steps issued together per row group

template <int RW, int KS>
__global__ __launch_bounds__(64 * KS) void read_probe_kernel(const char* __restrict__ w, int64_t rows,
                                                             uint32_t row_bytes, uint32_t* __restrict__ sink) {
  constexpr int G = RW / 4;
  const int lane = threadIdx.x & 63;
  const int wk = threadIdx.x >> 6;
  const int i4 = lane & 3, b4 = lane >> 2;
  const int64_t r0 = (int64_t)blockIdx.x * RW;
  const int64_t rows_valid = min((int64_t)RW, rows - r0);
  const rsrc_t rA = make_rsrc(w + r0 * row_bytes, (uint32_t)(rows_valid - 1) * row_bytes + row_bytes);
  const int steps = (int)((row_bytes + kStep4Bytes - 1) / kStep4Bytes);
  const int per_w = (steps + KS - 1) / KS;
  const int w0 = wk * per_w, w1 = min(steps, w0 + per_w);
  uint32_t fold = 0;
  for (int c0 = w0; c0 < w1; c0 += kProbeBatch) {
    u32x4_t A[G][kProbeBatch];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int s = 0; s < kProbeBatch; ++s) {
        const uint32_t k = (uint32_t)(c0 + s) * kStep4Bytes + (uint32_t)(b4 * kLaneBytes);
        const bool ok = c0 + s < w1 && k < row_bytes;
        A[g][s] = buf_load16<kAuxStream>(rA, ok ? (uint32_t)(4 * g + i4) * row_bytes + k : kOob);
      }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int s = 0; s < kProbeBatch; ++s) fold ^= A[g][s].x ^ A[g][s].y ^ A[g][s].z ^ A[g][s].w;
  }
  // every lane's fold is used (a store that depends on it), so no load is dead
  if (fold == 0x9e3779b9u || threadIdx.x == 0) sink[blockIdx.x] = fold;
}

__global__ void empty_probe_kernel() {}

// ---------------------------------------------------------------------------
// The M <= 4 skinny linear as first specified -- weights streamed with
// 128-bit loads, the workgroup's activations staged once in LDS, bf16 dot
// products on the VALU, lanes and waves reduced through LDS -- kept as a
// measurement probe beside thin_gemv4_kernel (4x4x4 MFMA, activations in
// registers), so the two designs run on the same shapes from the same build.
//   * grid: one workgroup per RW weight rows; its KS waves take the rows'
//     1 KB chunks (512 elements) in turn, U chunks per batch;
//   * load instruction: one row x 1 KB (lane l: bytes 16 l .. 16 l + 15 of
//     the chunk), non-temporal; all RW x U loads of a batch are issued
//     before its arithmetic;
//   * per 16-byte weight piece and token: 4 v_dot2_f32_bf16 against the
//     matching 16 bytes of the token's row, read from LDS (consecutive lanes,
//     consecutive 16 bytes: no bank conflicts);
//   * reduction: the wave's lanes by the lane-swap reduce-scatter
//     (reduce_lanes), then wave 0 adds the waves' totals in wave order from
//     LDS and rounds to bf16.
constexpr int kValuMT = 4;                  // tokens
constexpr int kValuMaxK = 6144;             // activation elements per token staged in LDS (48 KB)
constexpr int kValuChunk = 512;             // elements per row and load instruction

typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));

// The dwords are taken by subscript into scalars first: this compiler turns
// __builtin_bit_cast of a swizzle (a.y, a.z, ...) into a read of element 0.
SIMSD_DEV float dot8_bf16(u32x4_t a, u32x4_t b, float c) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t ai = a[i], bi = b[i];
    c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v_t, ai), __builtin_bit_cast(bf16x2v_t, bi), c, false);
  }
  return c;
}

template <int RW, int KS>
__global__ __launch_bounds__(64 * KS) void gemv_valu_probe_kernel(const char* __restrict__ x, int64_t sxm,
                                                                  const char* __restrict__ w, int64_t swn,
                                                                  char* __restrict__ y, int64_t sym, int M, int N,
                                                                  int K) {
  constexpr int U = 2;
  constexpr int NV = RW * kValuMT;                   // outputs per workgroup
  // dynamic LDS: the tokens' rows [kValuMT][K] bf16, then the waves' sums [KS][NV]
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int lane = threadIdx.x & 63;
  const int wk = threadIdx.x >> 6;
  const int64_t n0 = (int64_t)blockIdx.x * RW;
  const int k8 = K / 8;
  for (int i = threadIdx.x; i < kValuMT * k8; i += 64 * KS) {   // rows >= M as zeros
    const int m = i / k8, c = i % k8;
    const u32x4_t v = m < M ? *reinterpret_cast<const u32x4_t*>(x + ((int64_t)m * sxm + c * 8) * 2) : zero4();
    *reinterpret_cast<u32x4_t*>(smem + ((int64_t)m * K + c * 8) * 2) = v;
  }
  __syncthreads();
  const int rows_valid = (int)min((int64_t)RW, N - n0);
  const uint32_t row_b = (uint32_t)(swn * 2), Kb = (uint32_t)K * 2;
  const rsrc_t rw = make_rsrc(w + n0 * swn * 2, (uint32_t)(rows_valid - 1) * row_b + Kb);
  float acc[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) acc[v] = 0.f;
  const int nch = (K + kValuChunk - 1) / kValuChunk;
  for (int c0 = wk; c0 < nch; c0 += KS * U) {
    u32x4_t W[U][RW];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t k = (uint32_t)(c0 + u * KS) * (kValuChunk * 2) + lane * 16;
      const bool ok = c0 + u * KS < nch && k < Kb;
#pragma unroll
      for (int r = 0; r < RW; ++r) W[u][r] = buf_load16<kAuxStream>(rw, ok ? (uint32_t)r * row_b + k : kOob);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = (c0 + u * KS) * kValuChunk + lane * 8;
      const bool ok = c0 + u * KS < nch && k < K;
      u32x4_t X[kValuMT];
#pragma unroll
      for (int m = 0; m < kValuMT; ++m)
        X[m] = ok ? *reinterpret_cast<const u32x4_t*>(smem + ((int64_t)m * K + k) * 2) : zero4();
#pragma unroll
      for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int m = 0; m < kValuMT; ++m) acc[r * kValuMT + m] = dot8_bf16(W[u][r], X[m], acc[r * kValuMT + m]);
    }
  }
  // the wave's 64 lanes: lane l ends with output p + (l >> 4) * NV / 4 in acc[p]
  reduce_lanes<NV, 1>(acc);
  float* tot = reinterpret_cast<float*>(smem + kValuMT * K * 2);
  if ((lane & 15) == 0) {
#pragma unroll
    for (int p = 0; p < NV / 4; ++p) tot[wk * NV + p + (lane >> 4) * (NV / 4)] = acc[p];
  }
  __syncthreads();
  if (wk == 0 && lane < NV) {
    const int r = lane / kValuMT, m = lane % kValuMT;
    float s = 0.f;
    for (int v = 0; v < KS; ++v) s += tot[v * NV + lane];
    if (m < M && r < rows_valid) store_elem<kBF16>(y, (int64_t)m * sym + n0 + r, s);
  }
}

template <int RW>
void launch_valu(int waves, dim3 grid, const char* x, int64_t sxm, const char* w, int64_t swn, char* y, int64_t sym,
                 int M, int N, int K, hipStream_t st) {
  const size_t lds = (size_t)kValuMT * K * 2 + (size_t)waves * RW * kValuMT * 4;
  switch (waves) {
    case 2: hipLaunchKernelGGL((gemv_valu_probe_kernel<RW, 2>), grid, dim3(128), lds, st, x, sxm, w, swn, y, sym, M, N, K); break;
    case 8: hipLaunchKernelGGL((gemv_valu_probe_kernel<RW, 8>), grid, dim3(512), lds, st, x, sxm, w, swn, y, sym, M, N, K); break;
    default: hipLaunchKernelGGL((gemv_valu_probe_kernel<RW, 4>), grid, dim3(256), lds, st, x, sxm, w, swn, y, sym, M, N, K); break;
  }
}

template <int RW>
void launch_read(int waves, dim3 grid, const char* w, int64_t rows, uint32_t rb, uint32_t* sink, hipStream_t st) {
  switch (waves) {
    case 1: hipLaunchKernelGGL((read_probe_kernel<RW, 1>), grid, dim3(64), 0, st, w, rows, rb, sink); break;
    case 4: hipLaunchKernelGGL((read_probe_kernel<RW, 4>), grid, dim3(256), 0, st, w, rows, rb, sink); break;
    case 8: hipLaunchKernelGGL((read_probe_kernel<RW, 8>), grid, dim3(512), 0, st, w, rows, rb, sink); break;
    default: hipLaunchKernelGGL((read_probe_kernel<RW, 2>), grid, dim3(128), 0, st, w, rows, rb, sink); break;
  }
}

}  // namespace
}  // namespace simsd

using namespace simsd;

extern "C" int simsd_probe_empty(void* stream) {
  hipLaunchKernelGGL(empty_probe_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream));
  return check_launch("probe_empty");
}

extern "C" int simsd_probe_read(const void* w, int64_t rows, int64_t row_bytes, int rows_per_wg, int waves,
                                void* sink, int64_t sink_words, void* stream) {
  if (w == nullptr || sink == nullptr || rows < 1 || row_bytes < 16 || row_bytes % 16 != 0)
    return set_error("probe_read: need a buffer, rows >= 1 and row_bytes a positive multiple of 16");
  if ((reinterpret_cast<uintptr_t>(w) & 15u) != 0) return set_error("probe_read: buffer must be 16-byte aligned");
  if (rows_per_wg != 4 && rows_per_wg != 8 && rows_per_wg != 16)
    return set_error("probe_read: rows_per_wg must be 4, 8 or 16 (got %d)", rows_per_wg);
  if (waves != 1 && waves != 2 && waves != 4 && waves != 8)
    return set_error("probe_read: waves must be 1, 2, 4 or 8 (got %d)", waves);
  if (16 * row_bytes >= (int64_t)kOob) return set_error("probe_read: rows too long for 32-bit offsets");
  const int64_t wgs = (rows + rows_per_wg - 1) / rows_per_wg;
  if (sink_words < wgs) return set_error("probe_read: sink needs %lld words", (long long)wgs);
  const dim3 grid((unsigned)wgs);
  const char* p = static_cast<const char*>(w);
  uint32_t* s = static_cast<uint32_t*>(sink);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint32_t rb = (uint32_t)row_bytes;
  switch (rows_per_wg) {
    case 4: launch_read<4>(waves, grid, p, rows, rb, s, st); break;
    case 8: launch_read<8>(waves, grid, p, rows, rb, s, st); break;
    default: launch_read<16>(waves, grid, p, rows, rb, s, st); break;
  }
  return check_launch("probe_read");
}

extern "C" int simsd_probe_gemv_valu(const void* x, int64_t sxm, const void* w, int64_t swn, void* y, int64_t sym,
                                     int64_t M, int64_t N, int64_t K, int rows_per_wg, int waves, void* stream) {
  if (x == nullptr || w == nullptr || y == nullptr) return set_error("probe_gemv_valu: null pointer");
  if (M < 1 || M > kValuMT || N < 1 || K < 8 || K % 8 != 0 || K > kValuMaxK)
    return set_error("probe_gemv_valu: needs 1 <= M <= %d, N >= 1, K a multiple of 8 up to %d", kValuMT, kValuMaxK);
  if (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15u) != 0 || sxm % 8 != 0 || swn % 8 != 0 ||
      sxm < K || swn < K || sym < N)
    return set_error("probe_gemv_valu: rows must be 16-byte aligned and non-overlapping");
  if (rows_per_wg != 8 && rows_per_wg != 16) return set_error("probe_gemv_valu: rows_per_wg must be 8 or 16");
  if (waves != 2 && waves != 4 && waves != 8) return set_error("probe_gemv_valu: waves must be 2, 4 or 8");
  if ((int64_t)rows_per_wg * swn * 2 >= (int64_t)kOob) return set_error("probe_gemv_valu: rows too long for 32-bit offsets");
  const dim3 grid((unsigned)((N + rows_per_wg - 1) / rows_per_wg));
  const char* xp = static_cast<const char*>(x);
  const char* wp = static_cast<const char*>(w);
  char* yp = static_cast<char*>(y);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (rows_per_wg == 8) launch_valu<8>(waves, grid, xp, sxm, wp, swn, yp, sym, (int)M, (int)N, (int)K, st);
  else launch_valu<16>(waves, grid, xp, sxm, wp, swn, yp, sym, (int)M, (int)N, (int)K, st);
  return check_launch("probe_gemv_valu");
}
