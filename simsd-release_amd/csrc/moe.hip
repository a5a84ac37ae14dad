// Fused MoE step for gfx950: route top-k -> align -> grouped gate_up (+SiLU.mul)
// -> grouped down -> fp32 weighted combine (+ shared expert).
//
// Replaces kernels/moe_dispatch_fused.py:32-192 (reference): the Triton
// _grouped_gemm_kernel, the ~10 torch launches of _align (93-132) and the
// SiLU.mul / combine glue (182-192).  The routing gate itself is not in the
// reference operator; its semantics follow
// kernels/workspace/moe_dispatch/build_oracle.py:71-90 (top-k on the logits,
// sigmoid or softmax scores, optional renormalisation, routed scaling).
//
// Every launch has a grid fixed by (T, k, E, H, I) alone: tiles that the
// routing leaves empty exit at once, so the whole step can be captured in a
// hipGraph and replayed with new routings.
#include <math.h>

#include "simsd_common.hpp"
#include "simsd_kernels.h"

namespace simsd {

constexpr int kTile = 16;   // slots per tile (the reference's BLOCK_M)

// ============================================================ route top-k ===
// One wave per token; the E logits are spread over the 64 lanes.  Selection
// order is value descending, ties to the lower expert index.  Every reduction
// over the wave runs on lane permutes (wave_max / wave_sum / wave_argmax),
// none through LDS.  Lane j < k ends with pick j: its expert and weight.
template <int PL>
SIMSD_DEV void route_token(const float* row, int E, int k, int scoring, int renorm, float scale,
                           int& pick, float& weight) {
  const int lane = threadIdx.x & 63;
  float v[PL];
  uint64_t key[PL];   // (order bits of the logit) << 32 | ~expert; 0 once taken or past E
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < E ? row[e] : -INFINITY;
    key[i] = e < E ? ((uint64_t)float_order_bits(v[i]) << 32) | (uint32_t)~e : 0ull;
  }
  float mx = 0.f, denom = 1.f;
  if (scoring == SIMSD_SCORE_SOFTMAX) {
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PL; ++i)
      if (lane + 64 * i < E) m = fmaxf(m, v[i]);
    mx = wave_max(m);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < PL; ++i)
      if (lane + 64 * i < E) sum += expf(v[i] - mx);
    denom = wave_sum(sum);
  }
  float my_v = 0.f;
  int my_i = 0;
  for (int j = 0; j < k; ++j) {
    uint64_t best = key[0];
#pragma unroll
    for (int i = 1; i < PL; ++i) best = key[i] > best ? key[i] : best;
    best = wave_max_u64(best);
    const int bi = (int)~(uint32_t)best;   // a real entry: k <= E
#pragma unroll
    for (int i = 0; i < PL; ++i)
      if (bi == lane + 64 * i) key[i] = 0ull;
    if (lane == j) {
      my_i = bi;
      my_v = float_from_order_bits((uint32_t)(best >> 32));
    }
  }
  float sc = 0.f;
  if (lane < k) {
    sc = scoring == SIMSD_SCORE_SOFTMAX ? expf(my_v - mx) / denom : 1.f / (1.f + expf(-my_v));
  }
  if (renorm && k > 1) {
    const float tot = wave_sum(lane < k ? sc : 0.f);
    sc = sc / (tot + 1e-20f);
  }
  pick = my_i;
  weight = sc * scale;
}

template <int PL>
__global__ __launch_bounds__(256) void moe_route_kernel(const float* __restrict__ logits, int64_t T,
                                                        int E, int64_t stride_t, int k, int scoring,
                                                        int renorm, float scale,
                                                        int64_t* __restrict__ ids,
                                                        float* __restrict__ wout) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  int pick;
  float weight;
  route_token<PL>(logits + t * stride_t, E, k, scoring, renorm, scale, pick, weight);
  if (lane < k) {
    ids[t * k + lane] = (int64_t)pick;
    wout[t * k + lane] = weight;
  }
}

// ================================================================== align ===
// One workgroup.  counts by LDS histogram; exclusive scans of counts and of
// counts padded to 16; a stable counting sort walked by one wave in slot
// order (ballot-matched equal keys, rank = popcount of lower lanes); then the
// padded slot table and per-tile expert ids of kernels/moe_dispatch_fused.py:93-132.
constexpr int kAlignThreads = 1024;

SIMSD_DEV void block_exclusive_scan2(int a, int b, int& ea, int& eb, int& ta, int& tb,
                                     int* s_wa /* [32] */, int* s_wb /* [32] */) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const int ia = wave_inclusive_sum(a), ib = wave_inclusive_sum(b);
  if (lane == 63) { s_wa[wv] = ia; s_wb[wv] = ib; }
  __syncthreads();
  if (wv == 0) {
    const int xa = wave_inclusive_sum(lane < nw ? s_wa[lane] : 0);
    const int xb = wave_inclusive_sum(lane < nw ? s_wb[lane] : 0);
    if (lane < nw) { s_wa[lane] = xa; s_wb[lane] = xb; }
  }
  __syncthreads();
  const int base_a = wv > 0 ? s_wa[wv - 1] : 0, base_b = wv > 0 ? s_wb[wv - 1] : 0;
  ea = base_a + ia - a;
  eb = base_b + ib - b;
  ta = s_wa[nw - 1];
  tb = s_wb[nw - 1];
}

// tiles the picks can fill: min(E, M) + ceil(M / 16)
constexpr int kAlignMaxTiles = SIMSD_MOE_MAX_EXPERTS + SIMSD_MOE_MAX_SLOTS / kTile;

// LDS of the align step (one workgroup).
struct AlignLds {
  int key[SIMSD_MOE_MAX_SLOTS];         // expert of each slot, E for an invalid id
  int pos[SIMSD_MOE_MAX_EXPERTS + 1];   // histogram, then running position
  int off[SIMSD_MOE_MAX_EXPERTS + 1];   // exclusive scan of counts
  int pad[SIMSD_MOE_MAX_EXPERTS + 1];   // exclusive scan of padded counts
  int perm[SIMSD_MOE_MAX_SLOTS];
  int tile[kAlignMaxTiles];             // expert of each tile, E past the last
  int wa[32], wb[32];
};

// The align tables from sm.key[0..M): called by every thread of the
// workgroup after the keys are in LDS and visible (__syncthreads).
SIMSD_DEV void align_from_keys(AlignLds& sm, int M, int E, int num_tiles, int32_t* __restrict__ counts,
                               int32_t* __restrict__ offsets, int32_t* __restrict__ pad_offsets,
                               int32_t* __restrict__ perm, int32_t* __restrict__ slots,
                               int32_t* __restrict__ tile_expert) {
  const int tid = threadIdx.x;
  const int n_tab = min(num_tiles, kAlignMaxTiles);
  for (int e = tid; e <= E; e += kAlignThreads) sm.pos[e] = 0;
  for (int t = tid; t < n_tab; t += kAlignThreads) sm.tile[t] = E;
  __syncthreads();
  // 1. histogram; bucket E collects ids outside [0, E) (kept out of every group)
  for (int i = tid; i < M; i += kAlignThreads) atomicAdd(&sm.pos[sm.key[i]], 1);
  __syncthreads();
  // 2. scans (E <= 1024: one expert per thread)
  const int c = tid < E ? sm.pos[tid] : 0;
  const int pc = (c + kTile - 1) / kTile * kTile;
  int ec, epc, tc, tpc;
  block_exclusive_scan2(c, pc, ec, epc, tc, tpc, sm.wa, sm.wb);
  if (tid < E) {
    sm.off[tid] = ec;
    sm.pad[tid] = epc;
    counts[tid] = c;
    offsets[tid] = ec;
    pad_offsets[tid] = epc;
    // tile t is expert e's when pad[e] <= 16 t < pad[e + 1]
    for (int t = epc / kTile; t < (epc + pc) / kTile && t < n_tab; ++t) sm.tile[t] = tid;
  }
  if (tid == 0) {
    sm.off[E] = tc;
    sm.pad[E] = tpc;
    offsets[E] = tc;
    pad_offsets[E] = tpc;
  }
  __syncthreads();
  // 3. stable scatter, one wave, 64 slots at a time in slot order
  if (tid < 64) {
    const int lane = tid;
    for (int e = lane; e <= E; e += 64) sm.pos[e] = sm.off[e];   // bucket E starts at tc
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int key_bits = 1;
    while ((1 << key_bits) <= E + 1) ++key_bits;
    for (int base = 0; base < M; base += 64) {
      const int i = base + lane;
      const int key = i < M ? sm.key[i] + 1 : 0;   // 0: no slot; else bucket + 1
      uint64_t same = ~0ull;
      for (int bt = 0; bt < key_bits; ++bt) {
        const bool bit = (key >> bt) & 1;
        const uint64_t bb = __ballot(bit);
        same &= bit ? bb : ~bb;
      }
      const int rank = __popcll(same & lt_mask);
      const int leader = __ffsll((unsigned long long)same) - 1;
      int p = 0;
      if (key > 0) p = sm.pos[key - 1] + rank;
      if (key > 0 && lane == leader) sm.pos[key - 1] = p + __popcll(same);
      if (key > 0) sm.perm[p] = i;
    }
  }
  __syncthreads();
  // 4. outputs: the padded slot table a row per thread from the tile table
  // (tiles past it are E's)
  for (int p = tid; p < M; p += kAlignThreads) perm[p] = sm.perm[p];
  const int total_rows = num_tiles * kTile;
  for (int q = tid; q < total_rows; q += kAlignThreads) {
    const int t = q / kTile;
    const int e = t < n_tab ? sm.tile[t] : E;
    int slot = -1;
    if (e < E) {
      const int r = q - sm.pad[e];
      if (r < sm.off[e + 1] - sm.off[e]) slot = sm.perm[sm.off[e] + r];
    }
    slots[q] = slot;
    if (q % kTile == 0) tile_expert[t] = e;
  }
}

__global__ __launch_bounds__(kAlignThreads) void moe_align_kernel(
    const int64_t* __restrict__ ids, int M, int E, int num_tiles, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ pad_offsets, int32_t* __restrict__ perm,
    int32_t* __restrict__ slots, int32_t* __restrict__ tile_expert) {
  __shared__ AlignLds sm;
  for (int i = threadIdx.x; i < M; i += kAlignThreads) {
    const int64_t e = ids[i];
    sm.key[i] = (e >= 0 && e < E) ? (int)e : E;
  }
  __syncthreads();
  align_from_keys(sm, M, E, num_tiles, counts, offsets, pad_offsets, perm, slots, tile_expert);
}

// Route every token (one wave per token, 16 waves) and align the picks in
// the same workgroup: the keys never leave LDS and the step saves a launch.
template <int PL>
__global__ __launch_bounds__(kAlignThreads) void moe_route_align_kernel(
    const float* __restrict__ logits, int T, int E, int64_t stride_t, int k, int scoring, int renorm,
    float scale, int64_t* __restrict__ ids, float* __restrict__ wout, int num_tiles,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets, int32_t* __restrict__ pad_offsets,
    int32_t* __restrict__ perm, int32_t* __restrict__ slots, int32_t* __restrict__ tile_expert) {
  __shared__ AlignLds sm;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  for (int t = wv; t < T; t += kAlignThreads / 64) {
    int pick;
    float weight;
    route_token<PL>(logits + (int64_t)t * stride_t, E, k, scoring, renorm, scale, pick, weight);
    if (lane < k) {
      ids[(int64_t)t * k + lane] = (int64_t)pick;
      wout[(int64_t)t * k + lane] = weight;
      sm.key[t * k + lane] = pick;
    }
  }
  __syncthreads();
  align_from_keys(sm, T * k, E, num_tiles, counts, offsets, pad_offsets, perm, slots, tile_expert);
}

// Route and align for up to 128 picks (T*k <= 128): the tokens are routed
// as above, then one wave builds the counts, offsets and permutation with no
// further barrier -- the picks are 2 keys per lane, the histogram and scans
// live in that wave's LDS (its LDS operations complete in order), ranks among
// equal experts come from ballots -- and a tile -> expert table, written by
// each active expert's lane over its own tiles; after one barrier every
// thread fills padded rows of the slot table from it.  The same tables as
// align_from_keys.
constexpr int kSmallAlignSlots = 128;
// tiles the picks can fill: min(E, M) + ceil(M / 16) for M <= 128
constexpr int kSmallAlignTiles = kSmallAlignSlots + kSmallAlignSlots / kTile;

// Wave 0's part of moe_route_align_small_kernel: counts, offsets, the stable
// permutation and the tile -> expert table, from the M keys in key_sh.
SIMSD_DEV void small_align_wave(const int* key_sh, int* off_sh, int* pad_sh, int* h0_sh, int* perm_sh,
                                int* tile_sh, int M, int E, int n_tab, int32_t* __restrict__ counts,
                                int32_t* __restrict__ offsets, int32_t* __restrict__ pad_offsets,
                                int32_t* __restrict__ perm) {
  const int lane = threadIdx.x & 63;
  // lane holds slots lane (key a) and 64 + lane (key b); -1 = no slot
  const int ka = lane < M ? key_sh[lane] : -1;
  const int kb = 64 + lane < M ? key_sh[64 + lane] : -1;
  for (int e = lane; e < E; e += 64) {
    off_sh[e] = 0;
    h0_sh[e] = 0;
  }
  if (ka >= 0) {
    atomicAdd(&off_sh[ka], 1);
    atomicAdd(&h0_sh[ka], 1);
  }
  if (kb >= 0) atomicAdd(&off_sh[kb], 1);
  // exclusive scans of the counts and of the 16-padded counts; lane owns the
  // experts [lane * EPL, lane * EPL + EPL)
  const int EPL = (E + 63) / 64;
  int c_sum = 0, p_sum = 0;
  for (int q = 0; q < EPL; ++q) {
    const int e = lane * EPL + q;
    const int c = e < E ? off_sh[e] : 0;
    c_sum += c;
    p_sum += (c + kTile - 1) / kTile * kTile;
  }
  const int c_inc = wave_inclusive_sum(c_sum), p_inc = wave_inclusive_sum(p_sum);
  int c_run = c_inc - c_sum, p_run = p_inc - p_sum;
  for (int q = 0; q < EPL; ++q) {
    const int e = lane * EPL + q;
    if (e < E) {
      const int c = off_sh[e];
      counts[e] = c;
      offsets[e] = c_run;
      pad_offsets[e] = p_run;
      off_sh[e] = c_run;
      pad_sh[e] = p_run;
      c_run += c;
      p_run += (c + kTile - 1) / kTile * kTile;
    }
  }
  if (lane == 63) {
    offsets[E] = c_inc;
    pad_offsets[E] = p_inc;
    off_sh[E] = c_inc;
    pad_sh[E] = p_inc;
  }
  // stable order by expert: rank among equal keys in slot order
  int key_bits = 1;
  while ((1 << key_bits) < E) ++key_bits;
  const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  uint64_t sa = __ballot(ka >= 0), sb = __ballot(kb >= 0);
  for (int b = 0; b < key_bits; ++b) {
    const bool ba = (ka >> b) & 1, bb = (kb >> b) & 1;
    const uint64_t wa = __ballot(ba), wb = __ballot(bb);
    sa &= ba ? wa : ~wa;
    sb &= bb ? wb : ~wb;
  }
  if (ka >= 0) {
    const int p = off_sh[ka] + __popcll(sa & lt);
    perm[p] = lane;
    perm_sh[p] = lane;
  }
  if (kb >= 0) {
    const int p = off_sh[kb] + h0_sh[kb] + __popcll(sb & lt);
    perm[p] = 64 + lane;
    perm_sh[p] = 64 + lane;
  }
  // tile t is expert e's when pad[e] <= 16 t < pad[e + 1]: E everywhere,
  // then each active expert's lane over its own tiles (after the E writes:
  // one wave's LDS operations complete in order)
  for (int t = lane; t < n_tab; t += 64) tile_sh[t] = E;
  for (int q = 0; q < EPL; ++q) {
    const int e = lane * EPL + q;
    if (e < E)
      for (int t = pad_sh[e] / kTile; t < pad_sh[e + 1] / kTile && t < n_tab; ++t) tile_sh[t] = e;
  }
}

template <int PL>
__global__ __launch_bounds__(kAlignThreads) void moe_route_align_small_kernel(
    const float* __restrict__ logits, int T, int E, int64_t stride_t, int k, int scoring, int renorm,
    float scale, int64_t* __restrict__ ids, float* __restrict__ wout, int num_tiles,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets, int32_t* __restrict__ pad_offsets,
    int32_t* __restrict__ perm, int32_t* __restrict__ slots, int32_t* __restrict__ tile_expert) {
  __shared__ int key_sh[kSmallAlignSlots];
  __shared__ int off_sh[SIMSD_MOE_MAX_EXPERTS + 1];   // counts, then offsets
  __shared__ int pad_sh[SIMSD_MOE_MAX_EXPERTS + 1];   // padded offsets
  __shared__ int h0_sh[SIMSD_MOE_MAX_EXPERTS];        // counts among slots 0..63
  __shared__ int perm_sh[kSmallAlignSlots];
  __shared__ int tile_sh[kSmallAlignTiles];           // expert of each tile, E past the last
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  for (int t = wv; t < T; t += kAlignThreads / 64) {
    int pick;
    float weight;
    route_token<PL>(logits + (int64_t)t * stride_t, E, k, scoring, renorm, scale, pick, weight);
    if (lane < k) {
      ids[(int64_t)t * k + lane] = (int64_t)pick;
      wout[(int64_t)t * k + lane] = weight;
      key_sh[t * k + lane] = pick;
    }
  }
  __syncthreads();
  const int M = T * k;
  const int n_tab = min(num_tiles, kSmallAlignTiles);
  if (wv == 0) small_align_wave(key_sh, off_sh, pad_sh, h0_sh, perm_sh, tile_sh, M, E, n_tab, counts, offsets,
                                pad_offsets, perm);
  __syncthreads();
  // the padded slot table, a row per thread; tiles past the table's are E's
  for (int q = threadIdx.x; q < num_tiles * kTile; q += kAlignThreads) {
    const int t = q / kTile, r = q % kTile;
    const int e = t < n_tab ? tile_sh[t] : E;
    int slot = -1;
    if (e < E) {
      const int rr = t * kTile - pad_sh[e] + r;
      if (rr < off_sh[e + 1] - off_sh[e]) slot = perm_sh[off_sh[e] + rr];
    }
    slots[q] = slot;
    if (r == 0) tile_expert[t] = e;
  }
}

// ======================================================== grouped FFN ======
struct MoeArgs {
  const char* x;
  int64_t sxt, sxh;
  const char* wg;
  int64_t sge, sgi, sgh;
  const char* wu;
  int64_t sue, sui, suh;
  const char* wd;
  int64_t sde, sdh, sdi;
  // shared expert (nullable): gate/up [Is, H], down [H, Is]
  const char* shg;
  int64_t shg_i, shg_h;
  const char* shu;
  int64_t shu_i, shu_h;
  const char* shd;
  int64_t shd_h, shd_i;
  const int32_t* slots;
  const int32_t* tile_expert;
  const int64_t* ids;
  const float* topk_w;
  int64_t sidt, sidk, swt, swk;
  char* h;    // [M, I]  slot-major
  char* hs;   // [T, Is]
  char* y;    // [M, H]
  char* ys;   // [T, H]
  char* out;
  int64_t sot, soh;
  int64_t T, H, I, Is;
  int k, E, num_tiles, shared_tiles;
};

// Decode which rows a tile feeds: a routed tile (expert e, gathered slots) or a
// shared-expert tile (16 consecutive tokens).  Returns false for an empty tile.
struct TileRows {
  int e;          // expert, or -1 for the shared expert
  int64_t slot;   // this lane's slot (routed) or token (shared); -1 if none
  int64_t token;  // row of x
};

SIMSD_DEV bool decode_tile(const int32_t* tile_expert, const int32_t* slots, int num_tiles, int E, int k, int T,
                           int t, int r, TileRows& tr) {
  if (t < num_tiles) {
    const int e = tile_expert[t];
    if (e < 0 || e >= E) return false;
    const int s = slots[(int64_t)t * kTile + r];
    tr.e = e;
    tr.slot = s;
    tr.token = s >= 0 ? s / k : -1;
  } else {
    const int64_t tok = (int64_t)(t - num_tiles) * kTile + r;
    tr.e = -1;
    tr.slot = tok < T ? tok : -1;
    tr.token = tr.slot;
  }
  return true;
}

// The MoE kernels take the tile table and two pointers and two strides their
// first loads depend on as leading scalar arguments, which the build preloads
// into SGPRs; the rest of MoeArgs is read where it is used.
#define SIMSD_MOE_HOT const int32_t *__restrict__ tile_expert, const int32_t *__restrict__ slots, int num_tiles, \
    int E, int k, int T, const char *__restrict__ p0, const char *__restrict__ p1, int i0, int i1, MoeArgs a

SIMSD_DEV float silu_f32(float v) { return v / (1.f + expf(-v)); }

// gate_up: one workgroup = one tile x 16 intermediate columns; rows of W_gate
// and W_up are the two A blocks, the tile's 16 gathered x rows the B block;
// 4 waves split H.  Epilogue h = silu(g) * u with the reference's rounding
// points (g, u, silu(g) and h each rounded to the storage dtype).
#ifndef SIMSD_MOE_GU_U
#define SIMSD_MOE_GU_U 2   // 256-byte k chunks per load batch in gate_up
#endif
#ifndef SIMSD_MOE_DN_U
#define SIMSD_MOE_DN_U 4   // 256-byte k chunks per load batch in down
#endif

// p0, p1: w_gate, w_up; i0, i1: their expert strides (elements)
template <int DT, bool FAST>
__global__ __launch_bounds__(256) void moe_gate_up_kernel(SIMSD_MOE_HOT) {
  constexpr int ES = DTypeInfo<DT>::kSize;
  constexpr int KS = 4;
  __shared__ __attribute__((aligned(16))) char gu_tile[KS][FAST ? 32 * kLdsRow : 16];
  const int lane = threadIdx.x & 63, wk = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int t = blockIdx.x;
  const int64_t c0i = (int64_t)blockIdx.y * 16;   // first intermediate column
  TileRows tr;
  if (!decode_tile(tile_expert, slots, num_tiles, E, k, T, t, r, tr)) return;
  const bool shared = tr.e < 0;
  const int64_t II = shared ? a.Is : a.I;
  if (c0i >= II) return;
  const char* wbase[2];
  int64_t a_sn[2], a_sk[2];
  if (shared) {
    wbase[0] = a.shg;
    wbase[1] = a.shu;
    a_sn[0] = a.shg_i; a_sn[1] = a.shu_i;
    a_sk[0] = a.shg_h * ES;
    a_sk[1] = a.shu_h * ES;
  } else {
    wbase[0] = p0 + (int64_t)tr.e * i0 * ES;
    wbase[1] = p1 + (int64_t)tr.e * i1 * ES;
    a_sn[0] = a.sgi; a_sn[1] = a.sui;
    a_sk[0] = a.sgh * ES;
    a_sk[1] = a.suh * ES;
  }
  const int steps = (int)((a.H * ES + kStepBytes - 1) / kStepBytes);
  const int per_w = (steps + KS - 1) / KS;
  const int w0 = wk * per_w, w1 = min(steps, w0 + per_w);
  f32x4_t acc[2][1] = {{f32x4_t{0.f, 0.f, 0.f, 0.f}}, {f32x4_t{0.f, 0.f, 0.f, 0.f}}};
  if (FAST) {
    // descriptors: the expert's gate and up matrices, and all of x; rows past
    // II and empty slots read as zero.  Weights stream as 4 rows x 256 B per
    // load through the wave's LDS tile (accum_lds).
    const uint32_t Kb = (uint32_t)(a.H * ES);
    rsrc_t ra[2];
    uint32_t a_row0[2], a_snb[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      a_snb[b] = (uint32_t)(a_sn[b] * ES);
      ra[b] = make_rsrc(wbase[b], (uint32_t)(II - 1) * a_snb[b] + Kb);
      a_row0[b] = (uint32_t)c0i * a_snb[b];
    }
    const uint32_t sxt_b = (uint32_t)(a.sxt * ES);
    const rsrc_t rB = make_rsrc(a.x, (uint32_t)(T - 1) * sxt_b + Kb);
    const uint32_t boff[1] = {tr.token >= 0 ? (uint32_t)tr.token * sxt_b : 0u};
    const bool bok[1] = {tr.token >= 0};
    const int chunks = (int)((Kb + kStep4Bytes - 1) / kStep4Bytes);
    const int per = (chunks + KS - 1) / KS;
    const int c0 = wk * per, c1 = min(chunks, c0 + per);
    accum_lds<DT, 2, 1, SIMSD_MOE_GU_U>(ra, a_row0, a_snb, rB, boff, bok, c0, c1, Kb, gu_tile[wk], acc);
  } else {
    const int64_t i_row = min(c0i + r, II - 1);
    const char* arow[2] = {wbase[0] + i_row * a_sn[0] * ES, wbase[1] + i_row * a_sn[1] * ES};
    const char* brow[1] = {tr.token >= 0 ? a.x + tr.token * a.sxt * ES : nullptr};
    // both A blocks share one k-stride in the generic gather; use per-block calls
    const char* a0[1] = {arow[0]};
    const char* a1[1] = {arow[1]};
    f32x4_t c0[1][1] = {{acc[0][0]}}, c1[1][1] = {{acc[1][0]}};
    accum_generic<DT, 1, 1>(a0, a_sk[0], brow, a.sxh * ES, w0, w1, g, a.H, c0);
    accum_generic<DT, 1, 1>(a1, a_sk[1], brow, a.sxh * ES, w0, w1, g, a.H, c1);
    acc[0][0] = c0[0][0];
    acc[1][0] = c1[0][0];
  }
  __shared__ float red[(KS - 1) * 2 * 4 * 64];
  reduce_waves<KS, 2>(reinterpret_cast<f32x4_t(&)[2]>(acc), wk, lane, red);
  if (wk != 0 || tr.slot < 0) return;
  char* orow = shared ? a.hs + tr.slot * a.Is * ES : a.h + tr.slot * a.I * ES;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t i = c0i + 4 * g + j;
    if (i < II) {
      const float gv = round_to<DT>(acc[0][0][j]);
      const float uv = round_to<DT>(acc[1][0][j]);
      const float sv = round_to<DT>(silu_f32(gv));
      store_elem<DT>(orow, i, sv * uv);
    }
  }
}

// down: one workgroup = one tile x 64 output features; each of the 4 waves owns
// 16 rows of W_down over the whole I.
template <int DT, bool FAST>
// p0, p1: w_down and the routed h rows; i0: w_down's expert stride, i1 its
// row stride (elements)
__global__ __launch_bounds__(256) void moe_down_kernel(SIMSD_MOE_HOT) {
  constexpr int ES = DTypeInfo<DT>::kSize;
  __shared__ __attribute__((aligned(16))) char dn_tile[4][FAST ? 16 * kLdsRow : 16];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int t = blockIdx.x;
  const int64_t n0 = (int64_t)blockIdx.y * 64 + wv * 16;
  TileRows tr;
  if (!decode_tile(tile_expert, slots, num_tiles, E, k, T, t, r, tr)) return;
  const bool shared = tr.e < 0;
  if (n0 >= a.H) return;
  const int64_t II = shared ? a.Is : a.I;
  const char* wbase = shared ? a.shd : p0 + (int64_t)tr.e * i0 * ES;
  const int64_t a_sn = shared ? a.shd_h : (int64_t)i1;
  const int64_t a_sk = (shared ? a.shd_i : a.sdi) * ES;
  const char* hbase = shared ? a.hs : p1;   // slot-major (or token-major) h, row length II
  const int steps = (int)((II * ES + kStepBytes - 1) / kStepBytes);
  f32x4_t acc[1][1] = {{f32x4_t{0.f, 0.f, 0.f, 0.f}}};
  if (FAST) {
    const uint32_t Kb = (uint32_t)(II * ES);
    const uint32_t sn_b = (uint32_t)(a_sn * ES);
    const int64_t h_rows = shared ? (int64_t)T : (int64_t)T * k;
    const rsrc_t ra[1] = {make_rsrc(wbase, (uint32_t)(a.H - 1) * sn_b + Kb)};
    const uint32_t a_row0[1] = {(uint32_t)n0 * sn_b};
    const uint32_t a_snb[1] = {sn_b};
    const rsrc_t rB = make_rsrc(hbase, (uint32_t)h_rows * Kb);
    const uint32_t boff[1] = {tr.slot >= 0 ? (uint32_t)tr.slot * Kb : 0u};
    const bool bok[1] = {tr.slot >= 0};
    const int chunks = (int)((Kb + kStep4Bytes - 1) / kStep4Bytes);
    accum_lds<DT, 1, 1, SIMSD_MOE_DN_U>(ra, a_row0, a_snb, rB, boff, bok, 0, chunks, Kb, dn_tile[wv], acc);
  } else {
    const char* arow[1] = {wbase + min(n0 + r, a.H - 1) * a_sn * ES};
    const char* brow[1] = {tr.slot >= 0 ? hbase + tr.slot * II * ES : nullptr};
    accum_generic<DT, 1, 1>(arow, a_sk, brow, ES, 0, steps, g, II, acc);
  }
  if (tr.slot < 0) return;
  char* orow = shared ? a.ys + tr.slot * a.H * ES : a.y + tr.slot * a.H * ES;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t n = n0 + 4 * g + j;
    if (n < a.H) store_elem<DT>(orow, n, acc[0][0][j]);
  }
}

// combine: out[t] = dtype( sum_j fp32(y[t*k+j]) * w[t,j] ), summed in j order,
// then (shared expert) out = dtype(out + ys[t]).  The ids, weights and expert
// outputs of 8 picks are loaded before any is used (one round trip, not 8);
// rows of invalid ids are read but not added.
// p0, p1: the routed expert outputs y and the ids; i0: H (the tile table
// arguments are unused here)
template <int DT>
__global__ __launch_bounds__(256) void moe_combine_kernel(SIMSD_MOE_HOT) {
  constexpr int J = 8;
  const int64_t t = blockIdx.y;
  const int64_t h = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t H = i0;
  if (h >= H) return;
  const int64_t* ids = reinterpret_cast<const int64_t*>(p1);
  float acc = 0.f;
  for (int j0 = 0; j0 < k; j0 += J) {
    int64_t e[J];
    float wv[J], yv[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const bool in = j0 + j < k;
      e[j] = in ? ids[t * a.sidt + (j0 + j) * a.sidk] : -1;
      wv[j] = in ? a.topk_w[t * a.swt + (j0 + j) * a.swk] : 0.f;
      yv[j] = in ? load_elem<DT>(p0, (t * k + j0 + j) * H + h) : 0.f;
    }
#pragma unroll
    for (int j = 0; j < J; ++j)
      if (e[j] >= 0 && e[j] < E) acc = __fadd_rn(acc, __fmul_rn(yv[j], wv[j]));
  }
  float o = round_to<DT>(acc);
  if (a.shared_tiles > 0) o = o + load_elem<DT>(a.ys, t * a.H + h);
  store_elem<DT>(a.out, t * a.sot + h * a.soh, o);
}

// down + combine for a few tokens (T <= kSmallT).  One workgroup owns R = 4*G
// output features for every token; its W waves take the tiles round-robin
// (the shared expert last), at most UM per wave.  A tile's weight rows stream
// in the GEMV layout of thin_gemv4_kernel (4 rows x 256 contiguous bytes per
// load, tokens as the 4 columns of v_mfma_f32_4x4x4) and are reused for each
// set of 4 valid slots of the tile (one set unless a token picks an expert
// twice).  A wave first reads the descriptors of all its tiles (one round
// trip), then keeps two tiles' loads in flight.  The expert outputs, rounded
// to the dtype as moe_down_kernel stores them, meet in LDS; the combine of
// moe_combine_kernel then runs on them: one launch instead of two, and no
// [T*k, H] round trip through memory.
constexpr int kSmallT = 4;
#ifndef SIMSD_MOE_SMALL_NB
#define SIMSD_MOE_SMALL_NB 2
#endif
constexpr int kSmallNB = SIMSD_MOE_SMALL_NB;   // unit buffers in flight per wave
constexpr int kSmallSlots = 64;   // T * k limit of the LDS table

template <int DT, int G, int S>
struct SmallUnit {
  u32x4_t A[G][S];
  u32x4_t B[S];
};

template <int DT, int G, int S, int W, int UM>
// p0, p1: w_down and the routed h rows; i0: w_down's expert stride, i1 its
// row stride (elements)
__global__ __launch_bounds__(64 * W) void moe_down_combine_kernel(SIMSD_MOE_HOT) {
  constexpr int ES = DTypeInfo<DT>::kSize;
  constexpr int R = 4 * G;
  __shared__ float y_sh[kSmallSlots + kSmallT][R];   // [slot t*k + j | T*k + token][feature]
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int i4 = lane & 3, b4 = lane >> 2;
  const int64_t n0 = (int64_t)blockIdx.x * R;
  const int rows = (int)min((int64_t)R, a.H - n0);
  const int n_units = num_tiles + (a.shared_tiles > 0 ? 1 : 0);
  const int M = T * k;
  const uint32_t lane_k = (uint32_t)b4 * kLaneBytes;

  // descriptors of this wave's units: expert (-1 shared, -2 none) and the
  // lane's column in each set of 4 (a slot, or a token for the shared
  // expert), all read in the first round trip -- a set past the first is
  // used only when a token picked the expert twice, and reading it later
  // would put a dependent load between consecutive units
  constexpr int kSets = kTile / 4;
  int ue[UM], ucol[UM][kSets];
#pragma unroll
  for (int i = 0; i < UM; ++i) {
    const int u = wv + i * W;
    if (u < num_tiles) {
      const int e = tile_expert[u];
      ue[i] = (e >= 0 && e < E) ? e : -2;
#pragma unroll
      for (int cs = 0; cs < kSets; ++cs) ucol[i][cs] = slots[(int64_t)u * kTile + 4 * cs + i4];
    } else if (u < n_units) {
      ue[i] = -1;
      ucol[i][0] = i4 < T ? i4 : -1;
#pragma unroll
      for (int cs = 1; cs < kSets; ++cs) ucol[i][cs] = -1;
    } else {
      ue[i] = -2;
#pragma unroll
      for (int cs = 0; cs < kSets; ++cs) ucol[i][cs] = -1;
    }
  }
  auto w_rsrc = [&](int e, uint32_t& sn_b, uint32_t& Kb) {
    const bool shared = e < 0;
    Kb = (uint32_t)((shared ? a.Is : a.I) * ES);
    const int64_t sn = shared ? a.shd_h : (int64_t)i1;
    sn_b = (uint32_t)(sn * ES);
    const char* wb = (shared ? a.shd : p0 + (int64_t)e * i0 * ES) + n0 * sn * ES;
    return make_rsrc(wb, (uint32_t)(rows - 1) * sn_b + Kb);
  };
  auto h_rsrc = [&](int e, uint32_t Kb) {
    return make_rsrc(e < 0 ? a.hs : p1, (uint32_t)(e < 0 ? T : M) * Kb);
  };
  auto load_b = [&](const rsrc_t& rH, uint32_t Kb, int col, u32x4_t (&B)[S]) {
#pragma unroll
    for (int st = 0; st < S; ++st) {
      const uint32_t k = (uint32_t)st * kStep4Bytes + lane_k;
      B[st] = buf_load16<kAuxKeep>(rH, (col >= 0 && k < Kb) ? (uint32_t)col * Kb + k : kOob);
    }
  };
  auto issue = [&](int i, SmallUnit<DT, G, S>& U) {
    if (ue[i] == -2) return;
    uint32_t sn_b, Kb;
    const rsrc_t rW = w_rsrc(ue[i], sn_b, Kb);
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int st = 0; st < S; ++st) {
        const uint32_t k = (uint32_t)st * kStep4Bytes + lane_k;
        U.A[g][st] = buf_load16<kAuxStream>(rW, k < Kb ? (uint32_t)(4 * g + i4) * sn_b + k : kOob);
      }
    load_b(h_rsrc(ue[i], Kb), Kb, ucol[i][0], U.B);
  };
  // one column set: MFMAs, the 16 k blocks summed (lane bits 2..5), lanes
  // with bits 2..3 clear hold feature q0 + p of column i4
  auto finish = [&](const SmallUnit<DT, G, S>& U, const u32x4_t (&B)[S], int col, bool shared) {
    f32x4_t acc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      acc[g] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < S; ++st) {
        acc[g] = Mfma4<DT>::step(lo2(U.A[g][st]), lo2(B[st]), acc[g]);
        acc[g] = Mfma4<DT>::step(hi2(U.A[g][st]), hi2(B[st]), acc[g]);
      }
    }
    constexpr int NV = G * 4;
    float val[NV];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) val[g * 4 + v] = acc[g][v];
    reduce_lanes<NV, 4>(val);
    if (((lane >> 2) & 3) == 0 && col >= 0) {
      const int q0 = ((lane >> 5) & 1) * (NV / 2) + ((lane >> 4) & 1) * (NV / 4);
      const int row = shared ? M + col : col;
#pragma unroll
      for (int p = 0; p < NV / 4; ++p) y_sh[row][q0 + p] = round_to<DT>(val[p]);
    }
  };
  auto compute = [&](int i, const SmallUnit<DT, G, S>& U) {
    if (ue[i] == -2) return;
    const bool shared = ue[i] == -1;
    finish(U, U.B, ucol[i][0], shared);
    if (shared) return;
    // further sets of 4 slots: only when a token picked this expert twice
    uint32_t Kb = (uint32_t)(a.I * ES);
    const rsrc_t rH = h_rsrc(ue[i], Kb);
#pragma unroll
    for (int cs = 1; cs < kSets; ++cs) {
      const int col = ucol[i][cs];
      if (!__any(col >= 0)) break;       // slots fill a tile from the front
      u32x4_t B[S];
      load_b(rH, Kb, col, B);
      finish(U, B, col, false);
    }
  };

  // NB unit buffers used in turn: the loads of the next NB - 1 units are in
  // flight while a unit's arithmetic runs (every index is a constant after
  // unrolling, so the buffers stay in registers)
  constexpr int kNB = S <= 4 ? kSmallNB : 2;   // 8 k steps a unit: two buffers fill the registers
  constexpr int NB = kNB < UM ? kNB : UM;
  SmallUnit<DT, G, S> U[NB];
#pragma unroll
  for (int b = 0; b + 1 < NB; ++b) issue(b, U[b]);
#pragma unroll
  for (int i = 0; i < UM; ++i) {
    if (i + NB - 1 < UM) issue(i + NB - 1, U[(i + NB - 1) % NB]);
    compute(i, U[i % NB]);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < (int)a.T * R; e += 64 * W) {
    const int64_t t = e / R;
    const int f = e % R;
    if (f >= rows) continue;
    float acc = 0.f;
    for (int j = 0; j < a.k; ++j) {
      const int64_t id = a.ids[t * a.sidt + j * a.sidk];
      const float w = a.topk_w[t * a.swt + j * a.swk];
      if (id >= 0 && id < a.E) acc = __fadd_rn(acc, __fmul_rn(y_sh[t * a.k + j][f], w));
    }
    float o = round_to<DT>(acc);
    if (a.shared_tiles > 0) o = o + y_sh[M + t][f];
    store_elem<DT>(a.out, t * a.sot + (n0 + f) * a.soh, o);
  }
}

// ------------------------------------------------------------------ host side
namespace {

inline int esize_of(int dtype) { return dtype == kF32 ? 4 : 2; }
inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool row_ok(const void* base, int64_t row_stride, int64_t k_stride, int64_t K, int es) {
  return base != nullptr && al16(base) && k_stride == 1 && (row_stride * es) % 16 == 0 &&
         (K * es) % 16 == 0;
}
inline int64_t align256(int64_t n) { return (n + 255) / 256 * 256; }

struct MoeLayout {
  int64_t h, hs, y, ys, total;
};

MoeLayout moe_layout(int64_t T, int k, int64_t H, int64_t I, int64_t Is, int es) {
  MoeLayout L{};
  const int64_t M = T * k;
  L.h = 0;
  L.hs = L.h + align256(M * I * es);
  L.y = L.hs + align256(T * Is * es);
  L.ys = L.y + align256(M * H * es);
  L.total = L.ys + align256(T * H * es);
  return L;
}

// the fused down + combine: small-T steps whose h rows fit S 256-byte steps;
// W waves of at most UM tiles each
#ifndef SIMSD_MOE_SMALL_G
#define SIMSD_MOE_SMALL_G 2
#endif
#ifndef SIMSD_MOE_SMALL_W
#define SIMSD_MOE_SMALL_W 8
#endif
#ifndef SIMSD_MOE_SMALL_UM
#define SIMSD_MOE_SMALL_UM 5
#endif
constexpr int kSmallG = SIMSD_MOE_SMALL_G, kSmallW = SIMSD_MOE_SMALL_W, kSmallUM = SIMSD_MOE_SMALL_UM;
constexpr int kSmallUM8 = 10;   // the 8-step variant: 4 features per workgroup

template <int DT>
void launch_ffn(const MoeArgs& a, bool fast_gu, bool fast_dn, bool small, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  const int tiles = a.num_tiles + a.shared_tiles;
  const int64_t imax = a.I > a.Is ? a.I : a.Is;
  dim3 g1((unsigned)tiles, (unsigned)((imax + 15) / 16));
  const int E = a.E, k = a.k, T = (int)a.T, nt = a.num_tiles;
  if (fast_gu)
    hipLaunchKernelGGL((moe_gate_up_kernel<DT, true>), g1, dim3(256), 0, stream, a.tile_expert, a.slots, nt, E, k, T,
                       a.wg, a.wu, (int)a.sge, (int)a.sue, a);
  else
    hipLaunchKernelGGL((moe_gate_up_kernel<DT, false>), g1, dim3(256), 0, stream, a.tile_expert, a.slots, nt, E, k, T,
                       a.wg, a.wu, (int)a.sge, (int)a.sue, a);
  if constexpr (DT != kF32) {
    if (small) {
      constexpr int R = 4 * kSmallG;
      const dim3 gs((unsigned)((a.H + R - 1) / R));
      if (imax * DTypeInfo<DT>::kSize <= 4 * kStep4Bytes)
        hipLaunchKernelGGL((moe_down_combine_kernel<DT, kSmallG, 4, kSmallW, kSmallUM>), gs, dim3(64 * kSmallW), 0,
                           stream, a.tile_expert, a.slots, nt, E, k, T, a.wd, a.h, (int)a.sde, (int)a.sdh, a);
      else   // twice the k steps: 4 features per workgroup
        hipLaunchKernelGGL((moe_down_combine_kernel<DT, 1, 8, kSmallW, kSmallUM8>),
                           dim3((unsigned)((a.H + 3) / 4)), dim3(64 * kSmallW), 0, stream, a.tile_expert, a.slots, nt,
                           E, k, T, a.wd, a.h, (int)a.sde, (int)a.sdh, a);
      return;
    }
  }
  dim3 g2((unsigned)tiles, (unsigned)((a.H + 63) / 64));
  if (fast_dn)
    hipLaunchKernelGGL((moe_down_kernel<DT, true>), g2, dim3(256), 0, stream, a.tile_expert, a.slots, nt, E, k, T, a.wd,
                       a.h, (int)a.sde, (int)a.sdh, a);
  else
    hipLaunchKernelGGL((moe_down_kernel<DT, false>), g2, dim3(256), 0, stream, a.tile_expert, a.slots, nt, E, k, T,
                       a.wd, a.h, (int)a.sde, (int)a.sdh, a);
  dim3 g3((unsigned)((a.H + 255) / 256), (unsigned)a.T);
  hipLaunchKernelGGL((moe_combine_kernel<DT>), g3, dim3(256), 0, stream, a.tile_expert, a.slots, nt, E, k, T, a.y,
                     reinterpret_cast<const char*>(a.ids), (int)a.H, 0, a);
}

}  // namespace
}  // namespace simsd

using namespace simsd;

extern "C" int simsd_moe_route_topk(const float* logits, int64_t T, int64_t E, int64_t stride_t,
                                    int k, int scoring, int renorm, float scale, int64_t* ids_out,
                                    float* w_out, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (T < 0 || E <= 0 || E > SIMSD_MOE_MAX_EXPERTS)
    return set_error("moe_route_topk: need 0 < E <= %d (E=%lld)", SIMSD_MOE_MAX_EXPERTS, (long long)E);
  if (k <= 0 || k > 64 || k > E) return set_error("moe_route_topk: need 0 < k <= min(64, E) (k=%d)", k);
  if (scoring != SIMSD_SCORE_SOFTMAX && scoring != SIMSD_SCORE_SIGMOID)
    return set_error("moe_route_topk: unknown scoring %d", scoring);
  if (T == 0) return 0;
  if (logits == nullptr || ids_out == nullptr || w_out == nullptr)
    return set_error("moe_route_topk: null pointer");
  if (T > (int64_t)0x7fffffff * 4) return set_error("moe_route_topk: T too large");
  dim3 grid((unsigned)((T + 3) / 4));
  if (E <= 64) hipLaunchKernelGGL((moe_route_kernel<1>), grid, dim3(256), 0, stream, logits, T, (int)E, stride_t, k, scoring, renorm, scale, ids_out, w_out);
  else if (E <= 256) hipLaunchKernelGGL((moe_route_kernel<4>), grid, dim3(256), 0, stream, logits, T, (int)E, stride_t, k, scoring, renorm, scale, ids_out, w_out);
  else hipLaunchKernelGGL((moe_route_kernel<16>), grid, dim3(256), 0, stream, logits, T, (int)E, stride_t, k, scoring, renorm, scale, ids_out, w_out);
  return check_launch("moe_route_topk");
}

extern "C" int simsd_moe_num_tiles(int64_t M, int64_t E) {
  return (int)((M < E ? M : E) + (M + kTile - 1) / kTile);
}

extern "C" int simsd_moe_align(const int64_t* ids, int64_t M, int64_t E, int num_tiles,
                               int32_t* counts, int32_t* offsets, int32_t* pad_offsets,
                               int32_t* perm, int32_t* slots, int32_t* tile_expert,
                               void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (E <= 0 || E > SIMSD_MOE_MAX_EXPERTS)
    return set_error("moe_align: need 0 < E <= %d", SIMSD_MOE_MAX_EXPERTS);
  if (M < 0 || M > SIMSD_MOE_MAX_SLOTS)
    return set_error("moe_align: need 0 <= T*k <= %d (got %lld)", SIMSD_MOE_MAX_SLOTS, (long long)M);
  if (num_tiles < 0 || (int64_t)num_tiles * kTile > ((int64_t)1 << 30))
    return set_error("moe_align: bad num_tiles %d", num_tiles);
  if (counts == nullptr || offsets == nullptr || pad_offsets == nullptr || slots == nullptr ||
      tile_expert == nullptr || (M > 0 && (ids == nullptr || perm == nullptr)))
    return set_error("moe_align: null pointer");
  hipLaunchKernelGGL(moe_align_kernel, dim3(1), dim3(kAlignThreads), 0, stream, ids, (int)M, (int)E,
                     num_tiles, counts, offsets, pad_offsets, perm, slots, tile_expert);
  return check_launch("moe_align");
}

extern "C" int simsd_moe_route_align(const float* logits, int64_t T, int64_t E, int64_t stride_t,
                                     int k, int scoring, int renorm, float scale, int64_t* ids_out,
                                     float* w_out, int num_tiles, int32_t* counts, int32_t* offsets,
                                     int32_t* pad_offsets, int32_t* perm, int32_t* slots,
                                     int32_t* tile_expert, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (E <= 0 || E > SIMSD_MOE_MAX_EXPERTS)
    return set_error("moe_route_align: need 0 < E <= %d (E=%lld)", SIMSD_MOE_MAX_EXPERTS, (long long)E);
  if (k <= 0 || k > 64 || k > E) return set_error("moe_route_align: need 0 < k <= min(64, E) (k=%d)", k);
  if (scoring != SIMSD_SCORE_SOFTMAX && scoring != SIMSD_SCORE_SIGMOID)
    return set_error("moe_route_align: unknown scoring %d", scoring);
  if (T < 0 || T * k > SIMSD_MOE_MAX_SLOTS)
    return set_error("moe_route_align: need 0 <= T*k <= %d (got %lld)", SIMSD_MOE_MAX_SLOTS,
                     (long long)(T * k));
  if (num_tiles < 0 || (int64_t)num_tiles * kTile > ((int64_t)1 << 30))
    return set_error("moe_route_align: bad num_tiles %d", num_tiles);
  if (counts == nullptr || offsets == nullptr || pad_offsets == nullptr || slots == nullptr ||
      tile_expert == nullptr ||
      (T > 0 && (logits == nullptr || ids_out == nullptr || w_out == nullptr || perm == nullptr)))
    return set_error("moe_route_align: null pointer");
  const dim3 grid(1), block(kAlignThreads);
  if (T * k <= kSmallAlignSlots && T <= kAlignThreads / 64) {
    if (E <= 64)
      hipLaunchKernelGGL((moe_route_align_small_kernel<1>), grid, block, 0, stream, logits, (int)T, (int)E, stride_t,
                         k, scoring, renorm, scale, ids_out, w_out, num_tiles, counts, offsets, pad_offsets, perm,
                         slots, tile_expert);
    else if (E <= 256)
      hipLaunchKernelGGL((moe_route_align_small_kernel<4>), grid, block, 0, stream, logits, (int)T, (int)E, stride_t,
                         k, scoring, renorm, scale, ids_out, w_out, num_tiles, counts, offsets, pad_offsets, perm,
                         slots, tile_expert);
    else
      hipLaunchKernelGGL((moe_route_align_small_kernel<16>), grid, block, 0, stream, logits, (int)T, (int)E,
                         stride_t, k, scoring, renorm, scale, ids_out, w_out, num_tiles, counts, offsets,
                         pad_offsets, perm, slots, tile_expert);
    return check_launch("moe_route_align");
  }
  if (E <= 64)
    hipLaunchKernelGGL((moe_route_align_kernel<1>), grid, block, 0, stream, logits, (int)T, (int)E, stride_t, k,
                       scoring, renorm, scale, ids_out, w_out, num_tiles, counts, offsets, pad_offsets, perm,
                       slots, tile_expert);
  else if (E <= 256)
    hipLaunchKernelGGL((moe_route_align_kernel<4>), grid, block, 0, stream, logits, (int)T, (int)E, stride_t, k,
                       scoring, renorm, scale, ids_out, w_out, num_tiles, counts, offsets, pad_offsets, perm,
                       slots, tile_expert);
  else
    hipLaunchKernelGGL((moe_route_align_kernel<16>), grid, block, 0, stream, logits, (int)T, (int)E, stride_t, k,
                       scoring, renorm, scale, ids_out, w_out, num_tiles, counts, offsets, pad_offsets, perm,
                       slots, tile_expert);
  return check_launch("moe_route_align");
}

extern "C" int64_t simsd_moe_workspace_bytes(int64_t T, int k, int64_t H, int64_t I, int64_t Is,
                                             int dtype) {
  return moe_layout(T, k, H, I, Is, esize_of(dtype)).total;
}

extern "C" int simsd_moe_grouped_ffn(
    const void* x, int64_t sxt, int64_t sxh, const void* w_gate, int64_t sge, int64_t sgi,
    int64_t sgh, const void* w_up, int64_t sue, int64_t sui, int64_t suh, const void* w_down,
    int64_t sde, int64_t sdh, int64_t sdi, const void* sh_gate, int64_t shg_i, int64_t shg_h,
    const void* sh_up, int64_t shu_i, int64_t shu_h, const void* sh_down, int64_t shd_h,
    int64_t shd_i, int64_t Is, const int32_t* slots, const int32_t* tile_expert, int num_tiles,
    const int64_t* topk_ids, int64_t sidt, int64_t sidk, const float* topk_w, int64_t swt,
    int64_t swk, void* out, int64_t sot, int64_t soh, int64_t T, int k, int64_t E, int64_t H,
    int64_t I, int dtype, void* workspace, int64_t workspace_bytes, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (dtype != kBF16 && dtype != kF16 && dtype != kF32)
    return set_error("moe_grouped_ffn: unsupported dtype code %d", dtype);
  if (T < 0 || k <= 0 || E <= 0 || H <= 0 || I <= 0)
    return set_error("moe_grouped_ffn: bad sizes T=%lld k=%d E=%lld H=%lld I=%lld", (long long)T, k,
                     (long long)E, (long long)H, (long long)I);
  if (T == 0) return 0;
  const bool has_shared = sh_gate != nullptr;
  if (has_shared && (sh_up == nullptr || sh_down == nullptr || Is <= 0))
    return set_error("moe_grouped_ffn: shared expert needs gate, up, down and Is > 0");
  if (!has_shared) Is = 0;
  const int es = esize_of(dtype);
  const MoeLayout L = moe_layout(T, k, H, I, Is, es);
  if (workspace == nullptr || workspace_bytes < L.total || !al16(workspace))
    return set_error("moe_grouped_ffn: needs a 16-byte aligned %lld-byte workspace (got %lld)",
                     (long long)L.total, (long long)workspace_bytes);
  if (x == nullptr || w_gate == nullptr || w_up == nullptr || w_down == nullptr || slots == nullptr ||
      tile_expert == nullptr || topk_ids == nullptr || topk_w == nullptr || out == nullptr)
    return set_error("moe_grouped_ffn: null pointer");
  const int64_t shared_tiles = has_shared ? (T + kTile - 1) / kTile : 0;
  if (num_tiles + shared_tiles > 0x7fffffff) return set_error("moe_grouped_ffn: too many tiles");
  auto fits = [](int64_t v) { return v >= -0x7fffffffll && v <= 0x7fffffffll; };
  if (!fits(T) || !fits(H) || !fits(sge) || !fits(sue) || !fits(sde) || !fits(sdh))
    return set_error("moe_grouped_ffn: T, H and the expert / row strides must fit 31 bits");   // kernel arguments
  MoeArgs a{};
  a.x = static_cast<const char*>(x); a.sxt = sxt; a.sxh = sxh;
  a.wg = static_cast<const char*>(w_gate); a.sge = sge; a.sgi = sgi; a.sgh = sgh;
  a.wu = static_cast<const char*>(w_up); a.sue = sue; a.sui = sui; a.suh = suh;
  a.wd = static_cast<const char*>(w_down); a.sde = sde; a.sdh = sdh; a.sdi = sdi;
  a.shg = static_cast<const char*>(sh_gate); a.shg_i = shg_i; a.shg_h = shg_h;
  a.shu = static_cast<const char*>(sh_up); a.shu_i = shu_i; a.shu_h = shu_h;
  a.shd = static_cast<const char*>(sh_down); a.shd_h = shd_h; a.shd_i = shd_i;
  a.slots = slots; a.tile_expert = tile_expert;
  a.ids = topk_ids; a.sidt = sidt; a.sidk = sidk;
  a.topk_w = topk_w; a.swt = swt; a.swk = swk;
  char* ws = static_cast<char*>(workspace);
  a.h = ws + L.h; a.hs = ws + L.hs; a.y = ws + L.y; a.ys = ws + L.ys;
  a.out = static_cast<char*>(out); a.sot = sot; a.soh = soh;
  a.T = T; a.H = H; a.I = I; a.Is = Is;
  a.k = k; a.E = (int)E; a.num_tiles = num_tiles; a.shared_tiles = (int)shared_tiles;
  // 16-byte paths: every operand row K-contiguous, 16-byte aligned, K*es % 16 == 0,
  // and every buffer-descriptor extent addressable with 32-bit offsets.
  const int64_t lim = (int64_t)kOob;
  const int64_t Imax = I > Is ? I : Is;
  bool fast_gu = row_ok(x, sxt, sxh, H, es) && row_ok(w_gate, sgi, sgh, H, es) &&
                 row_ok(w_up, sui, suh, H, es) && (sge * es) % 16 == 0 && (sue * es) % 16 == 0 &&
                 sxt > 0 && sgi > 0 && sui > 0 && T * sxt * es < lim &&
                 (I + 16) * sgi * es < lim && (I + 16) * sui * es < lim;
  bool fast_dn = row_ok(w_down, sdh, sdi, I, es) && (sde * es) % 16 == 0 && sdh > 0 &&
                 (H + 16) * sdh * es < lim && T * k * Imax * es < lim;
  if (has_shared) {
    fast_gu = fast_gu && row_ok(sh_gate, shg_i, shg_h, H, es) && row_ok(sh_up, shu_i, shu_h, H, es) &&
              shg_i > 0 && shu_i > 0 && (Is + 16) * shg_i * es < lim && (Is + 16) * shu_i * es < lim;
    fast_dn = fast_dn && row_ok(sh_down, shd_h, shd_i, Is, es) && shd_h > 0 &&
              (H + 16) * shd_h * es < lim;
  }
  // a few tokens: down and combine in one launch (every operand row 16-byte
  // aligned, h rows within 8 load steps, the T*k slot outputs within LDS)
  const int64_t units = num_tiles + (has_shared ? 1 : 0);
  const bool small = fast_dn && dtype != kF32 && T <= kSmallT && T * k <= kSmallSlots &&
                     Imax * es <= 8 * kStep4Bytes && (sde * es) % 16 == 0 && (sdh * es) % 16 == 0 &&
                     (!has_shared || (shd_h * es) % 16 == 0) &&
                     units <= kSmallW * (Imax * es <= 4 * kStep4Bytes ? kSmallUM : kSmallUM8);
  switch (dtype) {
    case kBF16: launch_ffn<kBF16>(a, fast_gu, fast_dn, small, stream); break;
    case kF16: launch_ffn<kF16>(a, fast_gu, fast_dn, small, stream); break;
    default: launch_ffn<kF32>(a, fast_gu, fast_dn, false, stream); break;
  }
  return check_launch("moe_grouped_ffn");
}
