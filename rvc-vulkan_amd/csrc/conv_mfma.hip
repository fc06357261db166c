// Implicit-GEMM conv1d on CDNA4 fp32 matrix cores (v_mfma_f32_32x32x2_f32).
//
// out[b][co][i] = sum_{ci,k} W[k][ci][co] * act(x[b][ci][i*S + in_off + k*dil])
// viewed as a GEMM with M = C_out, N = output positions and a reduction over
// (ci, k).  One workgroup owns a BM x BN output tile.  For each chunk of
// BK*SK input channels it stages, in LDS,
//   * the input window x[ci0:ci0+BK*SK][i0+in_off : i0+in_off+BN+(K-1)*dil]
//     once -- every tap re-reads the same window at a shift of k*dil, so the
//     halo is loaded once per chunk instead of K times, and
//   * the packed weights W[0:K][ci0:ci0+BK*SK][co0:co0+BM] (float4 loads).
// The next chunk's global loads are issued into registers before the MFMAs
// of the current chunk, so their latency hides behind the matrix work; each
// thread's staging offsets and padding masks are computed once per tile and
// the masks applied when the registers are stored to LDS, so no wait for
// those loads sits in front of the MFMAs.  Inside a chunk the LDS operands of
// step s+1 are read before the MFMAs of step s are issued (two register sets,
// ordered with sched_group_barrier).  The large decoder tiles keep two
// staging buffers: the prefetched registers go into the idle buffer right
// behind the current chunk's MFMAs, leaving one barrier per chunk.
//
// Each wave computes a WM x WN sub-tile with (WM/32)*(WN/32) 32x32
// accumulators.  With SK > 1 the SK waves that share a sub-tile split the
// staged channels between them (intra-workgroup split-K, for GEMMs with few
// output columns) and their partial sums are added through LDS at the end.
// Per MFMA step (two input channels) lane l supplies
//   A = W[k][c + l/32][co_tile + l%32]         (row = co, k-index = ci)
//   B = xs[c + l/32][col_tile + l%32 + k*dil]  (k-index = ci, col = i)
// and the 16 accumulator registers r of lane l hold
//   row = (r%4) + 4*(l/32) + 8*(r/4), col = l%32.
//
// The fused epilogue: bias (and an optional second per-channel term), an
// optional residual and, for an accumulating launch without activation, the
// current output are the accumulators' starting values (loaded while the
// first chunk stages); at the end leaky-ReLU / ReLU / tanh / GELU is applied
// and the result combined into the output (store, accumulate, or
// accumulate-then-divide).  Output position
// i is written at i*out_step + out_off, which lets one phase of a polyphase
// ConvTranspose1d use the same kernel.  A launch may carry up to
// kMaxConvGroups independent convolutions with the same channel counts
// (grid z = group x batch): the three ResBlocks of a decoder stage, or all
// ConvTranspose phases, run as one grid.
#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <type_traits>

#include "internal.h"

namespace rvc {

typedef float floatx16 __attribute__((ext_vector_type(16)));

namespace {

__device__ __forceinline__ float apply_act(float v, int act, float slope) {
  if (act == ACT_LEAKY) return v >= 0.f ? v : v * slope;
  if (act == ACT_TANH) return tanhf(v);
  if (act == ACT_RELU) return fmaxf(v, 0.f);
  if (act == ACT_GELU) return gelu_as(v);
  if (act == ACT_SIGMOID) return sigmoid_as(v);
  return v;
}

// S: input stride (output i reads inputs from i*S), a template parameter so
// the staged window and the B-operand addressing fold it at compile time.
// KMAX: most taps of any group of the launch; it sizes the register
// prefetch of the weights (1 for the plain GEMMs of 1x1 convolutions, which
// then afford wide channel chunks).
template <int BM, int BN, int WM, int WN, int BK, int SK, int S = 1, int KMAX = kConvTapsMax, int NBUF = 1>
struct Cfg {
  static constexpr int NWM = BM / WM;
  static constexpr int NWN = BN / WN;
  static constexpr int NWAVES = NWM * NWN * SK;
  static constexpr int NT = NWAVES * 64;
  static constexpr int TM = WM / 32;
  static constexpr int TN = WN / 32;
  static constexpr int BKT = BK * SK;
  static constexpr int XWMAX = BN * S + (KMAX > 1 ? kConvHaloMax : 0);
  static constexpr int XPT = (BKT * XWMAX + NT - 1) / NT;
  static constexpr int W4ROW = BM / 4;
  static constexpr int WPT = (KMAX * BKT * W4ROW + NT - 1) / NT;
  static size_t lds_bytes(int K, int dil) {
    const int XW = BN * S + (K > 0 ? (K - 1) * dil : 0);
    const size_t stage = NBUF * sizeof(float) * ((size_t)BKT * XW + (size_t)K * BKT * BM);
    const size_t red = SK > 1 ? sizeof(float) * (size_t)(SK - 1) * NWM * NWN * TM * TN * 16 * 64 : 0;
    return stage > red ? stage : red;
  }
};

// At least two resident waves per SIMD (the 1x1 GEMM tiles fit three unaided):
// without the cap the compiler spends registers on the accumulator-start
// loads and drops the 128 x 128 tile to one wave per SIMD (measured 30 %
// slower).
template <int BM, int BN, int WM, int WN, int BK, int SK, int S, int KMAX, int NBUF>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * SK * 64)
__attribute__((amdgpu_waves_per_eu(KMAX == 1 ? 1 : 2)))
void conv1d_mfma_kernel(ConvLaunch a) {
  using C = Cfg<BM, BN, WM, WN, BK, SK, S, KMAX, NBUF>;
  constexpr int NT = C::NT, TM = C::TM, TN = C::TN, BKT = C::BKT;
  constexpr int XPT = C::XPT, WPT = C::WPT, W4ROW = C::W4ROW;
  static_assert(BK % 2 == 0 && BKT % 4 == 0, "channel chunk must be a multiple of 4");

  const int b = blockIdx.z % a.B;
  const int gi = (blockIdx.z / a.B) % a.n_groups;
  const int ks = blockIdx.z / (a.B * a.n_groups);  // channel split of a split-K launch
  const ConvGroup G = a.g[gi];                      // one set of scalar loads
  // Tile order: workgroups are dispatched x-fastest and dealt round-robin to
  // the 8 XCDs (each with its own L2).  The C_out tiles of one column tile
  // read the same input window, so they are mapped 8 dispatch slots apart --
  // onto the same XCD, close in time -- and the input comes from L2 once.
  int tx = blockIdx.x, ty = blockIdx.y;
  if (gridDim.y > 1) {
    const int nty = gridDim.y;
    const int lin = blockIdx.y * gridDim.x + blockIdx.x;
    const int full = (gridDim.x / 8) * 8 * nty;  // linear slots of whole 8-column groups
    if (lin < full) {
      tx = (lin / (8 * nty)) * 8 + lin % 8;
      ty = (lin / 8) % nty;
    } else {
      tx = (gridDim.x / 8) * 8 + (lin - full) / nty;
      ty = (lin - full) % nty;
    }
  }
  const int i0 = tx * BN;
  // input channels of this workgroup: all, or one split of a.ksplit
  const int csplit = a.ksplit > 1 ? a.csplit : a.C_in;
  const int ci_lo = ks * csplit;
  const int ci_hi = min(a.C_in, ci_lo + csplit);
  if (i0 >= G.n_out) return;  // uniform for the whole workgroup, before any barrier
  const int co0 = ty * BM;
  const int K = G.K;
  const int dil = G.dil;
  const int XW = BN * S + (K > 0 ? (K - 1) * dil : 0);

  // NBUF staging buffers of [BKT][XW] inputs then [K][BKT][BM] weights
  // (BKT*XW and K*BKT*BM are multiples of 4, so every weight block is
  // 16-byte aligned)
  extern __shared__ float smem[];
  const int stage_floats = BKT * XW + K * BKT * BM;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wk = wave / (C::NWM * C::NWN);
  const int wr = wave % (C::NWM * C::NWN);
  const int wm = wr % C::NWM;
  const int wn = wr / C::NWM;
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const float* xb = G.x + (long long)b * a.xb;

  floatx16 acc[TM][TN];
#pragma unroll
  for (int m = 0; m < TM; ++m)
#pragma unroll
    for (int n = 0; n < TN; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[m][n][r] = 0.f;

  const bool fold_out = G.combine == COMB_ADD && a.out_act == ACT_NONE;
  const float* bias2 = a.bias2 ? a.bias2 + (long long)b * a.bias2b : nullptr;
  float* ob = G.out + (long long)b * a.ob;
  const float* rb = G.res ? G.res + (long long)b * a.rb : nullptr;
  if (a.ksplit <= 1 && wk == 0) {
#pragma unroll
    for (int m = 0; m < TM; ++m)
#pragma unroll
      for (int n = 0; n < TN; ++n) {
        const int i = i0 + wn * WN + n * 32 + l32;
        if (i >= G.n_out) continue;
        const long long t = (long long)i * G.out_step + G.out_off;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int co = co0 + wm * WM + m * 32 + (r & 3) + 4 * half + 8 * (r >> 2);
          if (co >= a.C_out) continue;
          float v = G.bias ? G.bias[co] : 0.f;
          if (bias2) v = v + bias2[co];
          if (rb) v = v + rb[co * a.rc + t];
          if (fold_out) v = v + ob[co * a.oc + t];
          acc[m][n][r] = v;
        }
      }
  }

  // Staging map, fixed across chunks: element e of this thread stages x row
  // xr_[e] (channel within the chunk) at window column j -> global offset
  // xo[e] = xr_[e]*xc + t from the chunk's first channel (-1: padding), and
  // weight vector e -> offset wo[e] from the chunk's first channel row.
  const int nx = BKT * XW;
  const int nw4 = K * BKT * W4ROW;
  const int tbase = i0 * S + G.in_off;
  int xo[XPT], xr_[XPT];
#pragma unroll
  for (int e = 0; e < XPT; ++e) {
    const int idx = tid + e * NT;
    const int r = idx / XW;
    const int j = idx - r * XW;
    const int t = tbase + j;
    const bool ok = idx < nx && t >= 0 && t < a.L_in;
    xr_[e] = ok ? r : 1 << 30;
    xo[e] = ok ? (int)((long long)r * a.xc + t) : 0;
  }
  int wo[WPT], wr_[WPT];
#pragma unroll
  for (int e = 0; e < WPT; ++e) {
    const int idx = tid + e * NT;
    const int row = idx / W4ROW;
    const int c4 = idx - row * W4ROW;
    const int k = row / BKT;
    const int rr = row - k * BKT;
    // columns past C_out (rounded up to 4) are never stored: not loaded either, so a
    // group whose weights start inside a wider packed row stays inside it
    const bool ok = idx < nw4 && co0 + 4 * c4 < ((a.C_out + 3) & ~3);
    wr_[e] = ok ? rr : 1 << 30;
    wo[e] = ok ? (k * a.C_in + rr) * a.w_ld + co0 + 4 * c4 : 0;
  }

  float xv[XPT];
  float4 wreg[WPT];
  // gload only issues the loads (masked elements read a valid dummy address);
  // the masks are applied by lstore, after the MFMAs that hide the latency.
  auto gload = [&](int ci0) {
    const float* xc0 = xb + (long long)ci0 * a.xc;
    const float* wc0 = G.w + (long long)ci0 * a.w_ld;
    const int lim = ci_hi - ci0;
#pragma unroll
    for (int e = 0; e < XPT; ++e) xv[e] = xc0[xr_[e] < lim ? xo[e] : 0];
#pragma unroll
    for (int e = 0; e < WPT; ++e) wreg[e] = *reinterpret_cast<const float4*>(wc0 + (wr_[e] < lim ? wo[e] : 0));
  };
  auto lstore = [&](int ci0, int buf) {
    float* xs = smem + buf * stage_floats;
    float* ws = xs + BKT * XW;
    const int lim = ci_hi - ci0;
#pragma unroll
    for (int e = 0; e < XPT; ++e) {
      const int idx = tid + e * NT;
      if (idx < nx) {
        float v = xr_[e] < lim ? xv[e] : 0.f;
        if (a.in_act == ACT_LEAKY) v = v >= 0.f ? v : v * a.in_slope;
        xs[idx] = v;
      }
    }
#pragma unroll
    for (int e = 0; e < WPT; ++e) {
      const int idx = tid + e * NT;
      if (idx < nw4) reinterpret_cast<float4*>(ws)[idx] = wr_[e] < lim ? wreg[e] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };

  if (K > 0 && ci_hi > ci_lo) {
    const int nchunk = (ci_hi - ci_lo + BKT - 1) / BKT;
    gload(ci_lo);
    lstore(ci_lo, 0);
    __syncthreads();
    for (int c = 0; c < nchunk; ++c) {
      const bool more = c + 1 < nchunk;
      const int cn = ci_lo + (c + 1) * BKT;
      if (more) gload(cn);
      const int buf = NBUF > 1 ? (c & 1) : 0;
      const float* xs = smem + buf * stage_floats;
      const float* ws = xs + BKT * XW;
      // software-pipelined: the LDS operands of step s+1 are read before the
      // MFMAs of step s are issued (two register sets, chosen by step parity)
      const float* wbase = ws + (wk * BK + half) * BM + wm * WM + l32;
      const float* xbase = xs + (wk * BK + half) * XW + (wn * WN + l32) * S;
      float av[2][TM], bv[2][TN];
      auto lda = [&](int k, int q, int p) {
        const float* w_ = wbase + (k * BKT + 2 * q) * BM;
        const float* x_ = xbase + 2 * q * XW + k * dil;
#pragma unroll
        for (int m = 0; m < TM; ++m) av[p][m] = w_[m * 32];
#pragma unroll
        for (int n = 0; n < TN; ++n) bv[p][n] = x_[n * 32 * S];
      };
      static_assert((BK / 2) % 2 == 0 || BK == 2, "step parity must repeat per tap");
      lda(0, 0, 0);
      for (int k = 0; k < K; ++k) {
#pragma unroll
        for (int q = 0; q < BK / 2; ++q) {
          const int p = q & 1;
          if (q + 1 < BK / 2)
            lda(k, q + 1, p ^ 1);
          else
            lda(k + 1 < K ? k + 1 : k, 0, p ^ 1);  // last tap: a harmless re-read, no branch
#pragma unroll
          for (int m = 0; m < TM; ++m)
#pragma unroll
            for (int n = 0; n < TN; ++n)
              acc[m][n] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[p][m], bv[p][n], acc[m][n], 0, 0, 0);
          // keep the next step's LDS reads ahead of this step's MFMAs
          __builtin_amdgcn_sched_group_barrier(0x100, (TM + 1) / 2 + (TN + 1) / 2, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, TM * TN, 0);
        }
      }
      if constexpr (NBUF > 1) {
        // the other buffer was last read in chunk c - 1, which every wave
        // finished before the previous barrier: store into it right behind
        // this chunk's MFMAs, one barrier per chunk
        if (more) lstore(cn, buf ^ 1);
        __syncthreads();
      } else {
        __syncthreads();
        if (more) {
          lstore(cn, 0);
          __syncthreads();
        }
      }
    }
  }

  if constexpr (SK > 1) {
    // partial sums of waves wk > 0 -> LDS, added in wk order by wave wk == 0
    float* red = smem;
    constexpr int PER = TM * TN * 16 * 64;
    if (wk > 0) {
      float* dst = red + ((wk - 1) * (C::NWM * C::NWN) + wr) * PER;
#pragma unroll
      for (int m = 0; m < TM; ++m)
#pragma unroll
        for (int n = 0; n < TN; ++n)
#pragma unroll
          for (int r = 0; r < 16; ++r) dst[((m * TN + n) * 16 + r) * 64 + lane] = acc[m][n][r];
    }
    __syncthreads();
    if (wk > 0) return;
#pragma unroll
    for (int s = 1; s < SK; ++s) {
      const float* src = red + ((s - 1) * (C::NWM * C::NWN) + wr) * PER;
#pragma unroll
      for (int m = 0; m < TM; ++m)
#pragma unroll
        for (int n = 0; n < TN; ++n)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[m][n][r] += src[((m * TN + n) * 16 + r) * 64 + lane];
    }
  }

  if (a.ksplit > 1) {
    // split-K partial sums: part[ks][b][co][i]; splitk_reduce_kernel adds the
    // splits in order and applies the epilogue
    float* pp = a.part + (((long long)ks * a.B + b) * a.C_out) * G.n_out;
#pragma unroll
    for (int m = 0; m < TM; ++m)
#pragma unroll
      for (int n = 0; n < TN; ++n) {
        const int i = i0 + wn * WN + n * 32 + l32;
        if (i >= G.n_out) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int co = co0 + wm * WM + m * 32 + (r & 3) + 4 * half + 8 * (r >> 2);
          if (co < a.C_out) pp[(long long)co * G.n_out + i] = acc[m][n][r];
        }
      }
    return;
  }

  // ---- fused epilogue (bias / residual / accumulate target already in acc) ----
#pragma unroll
  for (int m = 0; m < TM; ++m) {
#pragma unroll
    for (int n = 0; n < TN; ++n) {
      const int i = i0 + wn * WN + n * 32 + l32;
      if (i >= G.n_out) continue;
      const long long t = (long long)i * G.out_step + G.out_off;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = (r & 3) + 4 * half + 8 * (r >> 2);
        const int co = co0 + wm * WM + m * 32 + row;
        if (co >= a.C_out) continue;
        float v = apply_act(acc[m][n][r], a.out_act, a.out_slope);
        float* o = ob + co * a.oc + t;
        if (G.combine == COMB_ADD && !fold_out) {
          v = *o + v;
        } else if (G.combine == COMB_ADD_DIV) {
          v = (*o + v) / a.div;
        }
        *o = v;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Persistent variant for the large decoder launches (stride 1, one channel
// split, STORE with an optional residual or ADD without one).  The grid is one
// workgroup per resident slot; work item j = (group, batch item, column tile,
// C_out tile) -- groups in launch order, which the decoder sets heaviest (most
// taps) first -- goes to workgroup j % gridDim.x, so every workgroup gets the
// same mix and the short items fill the end.  The (item, chunk) sequence of a
// workgroup is one software pipeline over two LDS buffers: the next item's
// first chunk is loaded behind the current item's last chunk, and the
// current item's residual (or, for ADD, the current output) is prefetched
// into registers during that last chunk, so neither the start of an item nor
// its epilogue waits on global memory.  The sum is (conv + bias) + residual,
// the reference's order, and depends only on the tile shape, never on which
// workgroup runs the item.
__device__ __forceinline__ void persist_tile(int lin, int n_tx, int n_ty, int& tx, int& ty) {
  // the one-shot kernel's XCD-aware order (C_out tiles of one column tile 8
  // items apart); with a grid that is a multiple of 8, item j runs on XCD j % 8
  if (n_ty > 1) {
    const int full = (n_tx / 8) * 8 * n_ty;
    if (lin < full) {
      tx = (lin / (8 * n_ty)) * 8 + lin % 8;
      ty = (lin / 8) % n_ty;
    } else {
      tx = (n_tx / 8) * 8 + (lin - full) / n_ty;
      ty = (lin - full) % n_ty;
    }
  } else {
    tx = lin;
    ty = 0;
  }
}

// FAM only names the instantiation (1: the three-group stored launches of
// the decoder ResBlocks), so profiles can tell them from the other launches
// of the same tile; the code is identical.
//
// DIRECT (launches whose input takes no activation): chunks are staged by
// direct-to-LDS buffer loads (lane i of a wave writes 4 or 16 bytes at the
// wave's LDS base + 4i or 16i; out-of-range lanes write 0), so the staged
// values never pass through registers.  A staging buffer then holds XREG
// floats of x (every thread's XPT values: the window of the widest halo) and
// WREG4 float4 of weights (the largest tap count's block); each wave waits
// for its own loads before the chunk's barrier.
//
// HC > 0: the staged input window's row stride is XWC = BN + HC, HC (16 or
// 64) at least the launch's largest halo (K - 1) dil, a compile-time
// constant: the MFMA operands' LDS addresses are then immediate offsets from
// one base per tap, and the staging offsets need no division by a runtime
// width.  HC = 0: the stride is the item's own window, BN + (K - 1) dil
// (fewer registers: the 32-row tiles, which measured faster this way).
template <int BM, int BN, int WM, int WN, int BK, int FAM, bool DIRECT = false, int HC = 0>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64)
__attribute__((amdgpu_waves_per_eu(4)))
void conv1d_mfma_persist_kernel(ConvLaunch a, int n_tx, int n_ty, int stage_floats, int cpx) {
  using C = Cfg<BM, BN, WM, WN, BK, 1, 1, kConvTapsMax, 2>;
  constexpr int NT = C::NT, TM = C::TM, TN = C::TN, BKT = BK;
  constexpr int WPT = C::WPT, W4ROW = C::W4ROW;
  static_assert(BK % 4 == 0 && (BK / 2) % 2 == 0, "channel chunk must be a multiple of 4");
  static_assert(HC <= kConvHaloMax, "halo class");
  constexpr int XWC = BN + (HC > 0 ? HC : kConvHaloMax);  // the widest staged row
  constexpr int XPT = (BKT * XWC + NT - 1) / NT;
  constexpr int XREG = HC > 0 ? (BKT * XWC + 63) / 64 * 64 : XPT * NT;  // whole waves of direct-to-LDS loads
  constexpr int WREG4 = kConvTapsMax * BKT * W4ROW;
  // the weight loads past WREG4 (the last round only) skip whole waves
  static_assert(!DIRECT || ((WPT - 1) * NT < WREG4 && WPT * NT >= WREG4 && (WREG4 - (WPT - 1) * NT) % 64 == 0),
                "direct staging: weight rounds");

  const int per_b = n_tx * n_ty;
  const int per_group = a.B * per_b;
  const int n_items = per_group * a.n_groups;
  int item = blockIdx.x;
  const int nchunk = a.C_in / BKT;  // the launcher requires C_in % BK == 0
  // Item scheduling.  Static: slot s runs items s, s + grid, ...  Dynamic
  // (a.queue): every workgroup starts on item blockIdx.x, then takes tickets
  // from the queue of its XCD slot class x = blockIdx.x % 8 (items x + 8 m,
  // heaviest group first), so a slot that drew light items takes more of
  // them and the items of one column tile still meet on one XCD.
  __shared__ int next_sh;
  const bool dyn = a.queue != nullptr && n_items > (int)gridDim.x;
  const int nq = gridDim.x % 8 == 0 ? 8 : 1;
  const int qx = blockIdx.x % nq;
  const int per_q = gridDim.x / nq;
  // First items in snake order: workgroup q of an XCD class (q = blockIdx / 8)
  // is dispatched to about CU q % cpx of that XCD, in round s = q / cpx; odd
  // rounds take their run of the heaviest-first item list in reverse, so a
  // CU that drew a heavy item in one round draws a light one in the next.
  // A permutation of [0, gridDim) that keeps blockIdx % 8, so the static
  // stride and the ticket queues still cover every item once.
  if (cpx > 0 && nq == 8) {
    const int q = (int)blockIdx.x / 8;
    const int r = q / cpx;
    if (r & 1) {
      const int n_r = min(cpx, per_q - r * cpx);
      item = (r * cpx + (n_r - 1 - (q - r * cpx))) * 8 + qx;
    }
  }
  if (item >= n_items) return;  // uniform for the whole workgroup, before any barrier

  extern __shared__ float smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % C::NWM;
  const int wn = wave / C::NWM;
  const int half = lane >> 5;
  const int l32 = lane & 31;

  // ---- staging side: the item whose chunks are being loaded.  Loads go
  // through buffer resources whose range is the chunk's part of the tensor:
  // padding and masked lanes carry an offset past that range and read 0. ----
  int s_gi = 0, s_b = 0, s_i0 = 0, s_co0 = 0, s_K = 1, s_dil = 1, s_XW = BN;
  const float* s_x = nullptr;
  const float* s_w = nullptr;
  unsigned xo[XPT], wo[WPT];  // byte offsets from the chunk's first channel
  constexpr unsigned kOut = 0x80000000u;
  auto setup = [&](int j) {
    s_gi = j / per_group;
    const int r = j - s_gi * per_group;
    s_b = r / per_b;
    int tx, ty;
    persist_tile(r - s_b * per_b, n_tx, n_ty, tx, ty);
    s_i0 = tx * BN;
    s_co0 = ty * BM;
    const ConvGroup& G = a.g[s_gi];
    s_K = G.K;
    s_dil = G.dil;
    s_XW = BN + (s_K - 1) * s_dil;
    s_x = G.x + (long long)s_b * a.xb;
    s_w = G.w;
    const int nw4 = s_K * BKT * W4ROW;
    const int tbase = s_i0 + G.in_off;
    if constexpr (HC > 0) {  // LDS row stride XWC, the item's window in its first s_XW columns
#pragma unroll
      for (int e = 0; e < XPT; ++e) {
        const int idx = tid + e * NT;
        const int row = idx / XWC;
        const int col = idx - row * XWC;
        const int t = tbase + col;
        xo[e] = row < BKT && col < s_XW && t >= 0 && t < a.L_in ? 4u * (unsigned)(row * (int)a.xc + t) : kOut;
      }
    } else {
      // LDS row stride s_XW: element idx = tid + e NT sits at row idx / s_XW,
      // column idx % s_XW.  NT <= BN <= s_XW, so element 0 is (0, tid) and each
      // step adds NT to the column, wrapping into the next row at most once:
      // no division by the runtime width.
      static_assert(HC > 0 || NT <= BN, "incremental staging offsets need NT <= BN");
      int row = 0, col = tid;
#pragma unroll
      for (int e = 0; e < XPT; ++e) {
        const int t = tbase + col;
        xo[e] = row < BKT && t >= 0 && t < a.L_in ? 4u * (unsigned)(row * (int)a.xc + t) : kOut;
        col += NT;
        if (col >= s_XW) {
          col -= s_XW;
          ++row;
        }
      }
    }
#pragma unroll
    for (int e = 0; e < WPT; ++e) {
      const int idx = tid + e * NT;
      const int row = idx / W4ROW;
      const int c4 = idx - row * W4ROW;
      const int k = row / BKT;
      const int rr = row - k * BKT;
      wo[e] = idx < nw4 && s_co0 + 4 * c4 < ((a.C_out + 3) & ~3)
                  ? 4u * (unsigned)((k * a.C_in + rr) * a.w_ld + s_co0 + 4 * c4)
                                                    : kOut;
    }
  };
  float xv[XPT];
  // Register staging of x (the leaky ReLU is applied on the way to LDS);
  // the weights need no transform and go straight into buffer nb's weight
  // block (direct-to-LDS loads, lanes past the item's taps masked).
  auto gload = [&](int ci0, int nb) {
    // ranges: rows ci0.. of x ((C_in - ci0 - 1) full rows + one of L_in), and
    // the weight rows k * C_in + ci0 + rr of every tap
    const unsigned xr = 4u * (unsigned)((a.C_in - ci0 - 1) * (int)a.xc + a.L_in);
    const unsigned wr = 4u * (unsigned)(((s_K - 1) * a.C_in + a.C_in - ci0) * a.w_ld);
    const __amdgpu_buffer_rsrc_t xrs = uniform_rsrc(s_x + (long long)ci0 * a.xc, xr);
    const __amdgpu_buffer_rsrc_t wrs = uniform_rsrc(s_w + (long long)ci0 * a.w_ld, wr);
#pragma unroll
    for (int e = 0; e < XPT; ++e) xv[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xrs, xo[e], 0, 0));
    float4* ws4 = reinterpret_cast<float4*>(smem + nb * stage_floats + BKT * (HC > 0 ? XWC : s_XW));
    const int nw4 = s_K * BKT * W4ROW;
    const int wb = wave * 64;
#pragma unroll
    for (int e = 0; e < WPT; ++e)
      if (tid + e * NT < nw4) buffer_load_lds_b128(wrs, ws4 + e * NT + wb, wo[e]);
  };
  auto gload_lds = [&](int ci0, int nb) {
    const unsigned xr = 4u * (unsigned)((a.C_in - ci0 - 1) * (int)a.xc + a.L_in);
    const unsigned wr = 4u * (unsigned)(((s_K - 1) * a.C_in + a.C_in - ci0) * a.w_ld);
    const __amdgpu_buffer_rsrc_t xrs = uniform_rsrc(s_x + (long long)ci0 * a.xc, xr);
    const __amdgpu_buffer_rsrc_t wrs = uniform_rsrc(s_w + (long long)ci0 * a.w_ld, wr);
    float* xs = smem + nb * stage_floats;
    float4* ws4 = reinterpret_cast<float4*>(xs + XREG);
    const int wb = wave * 64;
#pragma unroll
    for (int e = 0; e < XPT; ++e)
      if (HC == 0 || e + 1 < XPT || e * NT + wb < XREG) buffer_load_lds_b32(xrs, xs + e * NT + wb, xo[e]);
#pragma unroll
    for (int e = 0; e < WPT; ++e)
      if (e + 1 < WPT || e * NT + wb < WREG4) buffer_load_lds_b128(wrs, ws4 + e * NT + wb, wo[e]);
  };
  // every load of this wave (direct-to-LDS ones included) has landed
  auto wait_loads = [&]() { __builtin_amdgcn_s_waitcnt(0); };
  auto lstore = [&](int buf) {
    float* xs = smem + buf * stage_floats;
#pragma unroll
    for (int e = 0; e < XPT; ++e) {
      const int idx = tid + e * NT;
      if (idx < BKT * (HC > 0 ? XWC : s_XW)) {
        float v = xv[e];
        if (a.in_act == ACT_LEAKY) v = v >= 0.f ? v : v * a.in_slope;
        xs[idx] = v;
      }
    }
  };

  // MFMAs of one staged chunk (software-pipelined LDS operands, as in the
  // one-shot kernel)
  floatx16 acc[TM][TN];
  auto mfma_chunk = [&](int buf, int K, int dil, int XWr) {
    const int XW = HC > 0 ? XWC : XWr;  // the LDS row stride
    const float* xs = smem + buf * stage_floats;
    const float* ws = xs + (DIRECT ? XREG : BKT * XW);
    const float* wbase = ws + half * BM + wm * WM + l32;
    const float* xbase = xs + half * XW + wn * WN + l32;
    float av[4][TM], bv[4][TN];
    auto lda = [&](int k, int q, int p) {
      const float* w_ = wbase + (k * BKT + 2 * q) * BM;
      const float* x_ = xbase + 2 * q * XW + k * dil;
#pragma unroll
      for (int m = 0; m < TM; ++m) av[p][m] = w_[m * 32];
#pragma unroll
      for (int n = 0; n < TN; ++n) bv[p][n] = x_[n * 32];
    };
    // LDS operands run PD MFMA steps ahead of their use (three for the 32-row
    // tiles of stages 0 and 3, two for the 64-row tiles of stages 1-2, each
    // measured best for its tile), in a ring of four slots: with BK / 2 = 4
    // steps per tap the slot of step q is q itself, a compile-time index
    static_assert(BK / 2 == 4, "four steps per tap: the ring slot of a step is its q");
    constexpr int PD = BM == 32 ? 3 : 2;
    lda(0, 0, 0);
    lda(0, 1, 1);
    if (PD == 3) lda(0, 2, 2);
    // the 32 x 512 tiles (stage 3: four chunks per item, so staging and
    // epilogues are a large share) and the 64 x 256 tiles (stages 0-2) raise
    // the wave's issue priority while it runs the chunk's MFMAs: waves with
    // MFMAs ready win the arbitration over waves staging or storing (stage 3
    // 1.017 -> 0.98 ms; the 64 x 256 family +0.4 %, config 2 1116 -> 1120
    // audio-s/s; the 32 x 256 tiles measured 2-4 % slower with it)
    constexpr bool kPrio = BN == 512 || BM == 64;
    if constexpr (kPrio) __builtin_amdgcn_s_setprio(1);
    for (int k = 0; k < K; ++k) {
#pragma unroll
      for (int q = 0; q < BK / 2; ++q) {
        const int p = q;
        if (q + PD < BK / 2)
          lda(k, q + PD, q + PD);
        else
          lda(k + 1 < K ? k + 1 : k, q + PD - BK / 2, (q + PD) & 3);
#pragma unroll
        for (int m = 0; m < TM; ++m)
#pragma unroll
          for (int n = 0; n < TN; ++n)
            acc[m][n] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[p][m], bv[p][n], acc[m][n], 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, (TM + 1) / 2 + (TN + 1) / 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, TM * TN, 0);
      }
    }
    if constexpr (kPrio) __builtin_amdgcn_s_setprio(0);
  };

  setup(item);
  if (DIRECT) {
    gload_lds(0, 0);
    wait_loads();
  } else {
    gload(0, 0);
    lstore(0);
    wait_loads();
  }
  __syncthreads();
  int buf = 0;
  while (item < n_items) {
    // this workgroup's next item: the ticket is drawn now and published to
    // LDS behind the first chunk's MFMAs (its round trip overlaps them), read
    // by every thread after that chunk's barrier
    unsigned tk = 0;
    if (tid == 0 && dyn) tk = atomicAdd(a.queue + qx, 1u);
    auto publish = [&]() {
      if (tid == 0) next_sh = dyn ? qx + nq * (per_q + (int)tk) : item + (int)gridDim.x;
    };
    if (nchunk == 1) {
      publish();
      __syncthreads();
    }
    // the current item's geometry, kept before setup() moves on to the next
    const int c_gi = s_gi, c_b = s_b, c_i0 = s_i0, c_co0 = s_co0, c_K = s_K, c_dil = s_dil, c_XW = s_XW;
#pragma unroll
    for (int m = 0; m < TM; ++m)
#pragma unroll
      for (int n = 0; n < TN; ++n)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[m][n][r] = 0.f;
    // every chunk but the last: prefetch the next chunk of this item.  The
    // other buffer was last read in the previous chunk, which every wave
    // finished before the previous barrier.
    for (int c = 0; c + 1 < nchunk; ++c) {
      if (DIRECT)
        gload_lds((c + 1) * BKT, buf ^ 1);
      else
        gload((c + 1) * BKT, buf ^ 1);
      mfma_chunk(buf, c_K, c_dil, c_XW);
      if (!DIRECT) lstore(buf ^ 1);
      wait_loads();
      if (c == 0) publish();
      __syncthreads();
      buf ^= 1;
    }
    // the last chunk: prefetch the next item's first chunk and this item's
    // epilogue operand (the residual, or the current output for ADD)
    // the same value in every lane: readfirstlane tells the compiler so, and
    // the next item's geometry, pointers and buffer resources stay scalar
    const int next = __builtin_amdgcn_readfirstlane(next_sh);
    const bool more = next < n_items;
    if (more) {
      setup(next);
      if (DIRECT)
        gload_lds(0, buf ^ 1);
      else
        gload(0, buf ^ 1);
    }
    // Epilogue addressing through buffer resources over this batch item's
    // output / residual: lane offset (co_l, t) per column, the row within the
    // lane's 16 accumulator rows as a uniform offset; columns past n_out get
    // an out-of-range offset, so their loads read 0 and their stores drop.
    const ConvGroup& G = a.g[c_gi];
    const bool res = G.res != nullptr;
    const bool add = G.combine == COMB_ADD;
    const int co_l = c_co0 + wm * WM + 4 * half;
    const __amdgpu_buffer_rsrc_t ors = uniform_rsrc(G.out + (long long)c_b * a.ob, 4u * (unsigned)(a.C_out * (int)a.oc));
    const __amdgpu_buffer_rsrc_t prs =
        res ? uniform_rsrc(G.res + (long long)c_b * a.rb, 4u * (unsigned)(a.C_out * (int)a.rc)) : ors;
    const int pc = res ? (int)a.rc : (int)a.oc;
    unsigned ooff[TN], poff[TN];
#pragma unroll
    for (int n = 0; n < TN; ++n) {
      const int i = c_i0 + wn * WN + n * 32 + l32;
      const int t = i * G.out_step + G.out_off;
      const bool ok = i < G.n_out;
      ooff[n] = ok ? 4u * (unsigned)(co_l * (int)a.oc + t) : kOut;
      poff[n] = ok ? 4u * (unsigned)(co_l * pc + t) : kOut;
    }
    float pre[TM][TN][16];
    if (res || add) {
#pragma unroll
      for (int m = 0; m < TM; ++m)
#pragma unroll
        for (int n = 0; n < TN; ++n)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int roff = m * 32 + (r & 3) + 8 * (r >> 2);
            pre[m][n][r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(prs, poff[n], 4 * roff * pc, 0));
          }
    }
    mfma_chunk(buf, c_K, c_dil, c_XW);
    if (!DIRECT && more) lstore(buf ^ 1);
    wait_loads();
    __syncthreads();
    buf ^= 1;

    // ---- epilogue: ((acc + bias) [+ res]) -> act -> [pre +] -> store ----
    // The bias goes through a buffer resource (range 0 without a bias: every
    // load reads 0 and no lane branches), all its loads in flight together.
    // The decoder's ResBlock launches (a bias, STORE, no activation or the
    // leaky ReLU, with or without a residual) take a path with those choices
    // made once per item: two adds, or an add and the leaky ReLU, per value.
    const bool hb = G.bias != nullptr;
    const __amdgpu_buffer_rsrc_t brs = uniform_rsrc(G.bias, hb ? 4u * (unsigned)a.C_out : 0u);
    auto epilogue = [&](auto fast, auto fres, auto fleaky) {
#pragma unroll
      for (int m = 0; m < TM; ++m) {
        float bias[16];
#pragma unroll
        for (int r = 0; r < 16; ++r)
          bias[r] = __builtin_bit_cast(
              float, __builtin_amdgcn_raw_buffer_load_b32(brs, 4u * (unsigned)co_l, 4 * (m * 32 + (r & 3) + 8 * (r >> 2)), 0));
#pragma unroll
        for (int n = 0; n < TN; ++n)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int roff = m * 32 + (r & 3) + 8 * (r >> 2);
            float v = acc[m][n][r];
            if constexpr (decltype(fast)::value) {
              v = v + bias[r];
              if constexpr (decltype(fres)::value) v = v + pre[m][n][r];
              if constexpr (decltype(fleaky)::value) v = v >= 0.f ? v : v * a.out_slope;
            } else {
              if (hb) v = v + bias[r];
              if (res) v = v + pre[m][n][r];
              v = apply_act(v, a.out_act, a.out_slope);
              if (add) v = pre[m][n][r] + v;
            }
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), ors, ooff[n], 4 * roff * (int)a.oc, 0);
          }
      }
    };
    using T = std::true_type;
    using F = std::false_type;
    if (hb && !add && a.out_act == ACT_NONE) {
      if (res)
        epilogue(T{}, T{}, F{});
      else
        epilogue(T{}, F{}, F{});
    } else if (hb && !add && !res && a.out_act == ACT_LEAKY) {
      epilogue(T{}, F{}, T{});
    } else {
      epilogue(F{}, F{}, F{});
    }
    item = next;
  }
  // the last workgroup to finish (every other one has drawn its final ticket)
  // clears the counters for the next launch on this buffer
  if (dyn && tid == 0 && atomicAdd(a.queue + 8, 1u) == gridDim.x - 1)
    for (int i = 0; i < 9; ++i) __hip_atomic_store(a.queue + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Small convolutions (enc_p / flow at a few thousand frames).  One workgroup
// forms a 32 x BN output tile over the WHOLE reduction: its four waves each
// take a quarter of the input channels of every staged chunk, accumulate the
// full tile, and the quarters are added through LDS in wave order
// (((q0 + q1) + q2) + q3) -- one launch and no partial-sum tensor, where the
// split-K path writes and re-reads every split's partial tile.

// The shared epilogue: each of the NW waves stores its 32 x BN accumulators
// to red [wave][n][r][lane], the partial tiles are added in wave order, and
// thread tid forms column i0 + tid % BN of tile rows tid / BN + RS * k.  Every global operand is loaded (buffer loads, rows and
// columns out of range masked to the out-of-range offset) before the first
// use.  Plain: out = combine(act(v + bias (+ bias2) (+ residual))), the
// split-K reduce's order (combine COMB_SUB, out = out - that, only here).  WaveNet gate (gate = true): tile rows [0, 16) are
// channels cb + r, rows [16, 32) channels H + cb + r - 16, and
// out[c] = tanh(v_c + g_c) * sigmoid(v_{H+c} + g_{H+c}) for the 16 channels
// (v including the bias), g per batch item.
// Mean and 1 / den of a LayerNorm over C channels for column i0 + tid % BN,
// from the float64 (sum, sum of squares) of ntile 32-row tiles, double2
// [B][ntile][L] (ConvLaunch::stat_out).  NP = NT / BN threads per column:
// thread (p, col) adds tiles p, p + NP, ... with all its loads in flight,
// then one thread adds the NP partials in p order -- a fixed grouping, so
// the result depends on the statistics only.  mean = S / C, var = (Q - S *
// mean) / C, den = sqrt(var + eps) (the LayerNorm kernels' formulas with the
// two passes folded into the sums).  scratch: NT double2 + 2 BN floats of
// LDS; two barriers, every thread of the workgroup calls it.  Columns past L
// get 0, 0.
template <int NT, int BN>
__device__ __forceinline__ void ln_column_stats(const double* stat, int ntile, int C, int L, float eps, int b, int i0,
                                                float* scratch, float& mu, float& rd) {
  constexpr int NP = NT / BN;
  constexpr int kMaxPer = 4;  // tiles per thread: ntile <= NP * kMaxPer (checked by the launcher)
  const int tid = threadIdx.x;
  const int col = tid % BN, p = tid / BN;
  const int i = i0 + col;
  const bool icol = i < L;
  double2* part = reinterpret_cast<double2*>(scratch);
  float* out = reinterpret_cast<float*>(part + NT);
  const double2* st = reinterpret_cast<const double2*>(stat) + (long long)b * ntile * L + i;
  double2 v[kMaxPer];
#pragma unroll
  for (int u = 0; u < kMaxPer; ++u) {
    const int t = p + NP * u;
    v[u] = icol && t < ntile ? st[(long long)t * L] : make_double2(0.0, 0.0);
  }
  double S = 0.0, Q = 0.0;
#pragma unroll
  for (int u = 0; u < kMaxPer; ++u) {
    S += v[u].x;
    Q += v[u].y;
  }
  part[tid] = make_double2(S, Q);
  __syncthreads();
  if (tid < BN) {
    S = 0.0;
    Q = 0.0;
    for (int q = 0; q < NP; ++q) {
      const double2 w = part[q * BN + tid];
      S += w.x;
      Q += w.y;
    }
    const double md = S / C;
    out[tid] = (float)md;
    out[BN + tid] = 1.0f / sqrtf((float)(fmax(Q - S * md, 0.0) / C) + eps);
  }
  __syncthreads();
  mu = icol ? out[col] : 0.f;
  rd = icol ? out[BN + col] : 0.f;
  __syncthreads();  // the scratch is free again
}

template <int BN, int NW = 4>
__device__ __forceinline__ void small_conv_epilogue(const ConvLaunch& a, const ConvGroup& G, int b, int i0, int co0,
                                                    bool gate, const floatx16 (&acc)[BN / 32], float* red, float rs_mu,
                                                    float rs_rd, int split = -1) {
  constexpr int TN = BN / 32;
  constexpr int RS = 64 * NW / BN;
  constexpr int KO = 32 * BN / (64 * NW);
  constexpr unsigned kOut = 0x80000000u;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  __syncthreads();  // the staged operands are dead; the LDS now takes the quarters
#pragma unroll
  for (int n = 0; n < TN; ++n)
#pragma unroll
    for (int r = 0; r < 16; ++r) red[((wave * TN + n) * 16 + r) * 64 + lane] = acc[n][r];
  __syncthreads();

  const int H = a.post_H;
  const int col = tid % BN;
  const int i = i0 + col;
  const int n = col >> 5;
  const int c32 = col & 31;
  const bool icol = i < G.n_out;
  float v[KO];
  unsigned bo[KO], oo[KO], ro[KO];
#pragma unroll
  for (int k = 0; k < KO; ++k) {
    const int row = tid / BN + k * RS;
    const int r = (row >> 3) * 4 + (row & 3);
    const int ln = c32 + 32 * ((row >> 2) & 1);
    float t = red[(n * 16 + r) * 64 + ln];
#pragma unroll
    for (int w = 1; w < NW; ++w) t = t + red[((w * TN + n) * 16 + r) * 64 + ln];
    v[k] = t;
    const int co = gate ? (row < 16 ? co0 + row : H + co0 + row - 16) : co0 + row;
    const bool ok = icol && co < a.C_out;
    bo[k] = ok ? 4u * (unsigned)co : kOut;
    oo[k] = ok ? 4u * (unsigned)(co * (int)a.oc + i) : kOut;
    ro[k] = ok ? 4u * (unsigned)(co * (int)a.rc + i) : kOut;
  }
  if (split >= 0) {
    // one split of a split reduction: the raw partial tile to
    // part[split][b][C_out][n_out]; splitk_small_reduce_kernel forms the output
    const long long pb = ((long long)split * a.B + b) * a.C_out * G.n_out;
    const __amdgpu_buffer_rsrc_t prs = uniform_rsrc(a.part + pb, 4u * (unsigned)(a.C_out * G.n_out));
#pragma unroll
    for (int k = 0; k < KO; ++k) {
      const int row = tid / BN + k * RS;
      const unsigned po = icol && co0 + row < a.C_out ? 4u * (unsigned)((co0 + row) * G.n_out + i) : kOut;
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v[k]), prs, po, 0, 0);
    }
    return;
  }
  float bv[KO];
  if (G.bias) {
    const __amdgpu_buffer_rsrc_t rs = uniform_rsrc(G.bias, 4u * (unsigned)a.C_out);
#pragma unroll
    for (int k = 0; k < KO; ++k) bv[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, bo[k], 0, 0));
  }
  float* ob = G.out + (long long)b * a.ob;
  if (gate) {
    // rows k < KO / 2 are the tanh channels, rows k + KO / 2 their sigmoid partners
    const __amdgpu_buffer_rsrc_t ors = uniform_rsrc(ob, 4u * (unsigned)((H - 1) * (int)a.oc + G.n_out));
    const __amdgpu_buffer_rsrc_t grs = uniform_rsrc(a.post_g + (long long)b * a.post_gb, 8u * (unsigned)H);
    float gv[KO];
#pragma unroll
    for (int k = 0; k < KO; ++k) gv[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(grs, bo[k], 0, 0));
#pragma unroll
    for (int k = 0; k < KO / 2; ++k) {
      float v1 = v[k], v2 = v[k + KO / 2];
      if (G.bias) {
        v1 = v1 + bv[k];
        v2 = v2 + bv[k + KO / 2];
      }
      const float t = tanhf(v1 + gv[k]) * sigmoid_as(v2 + gv[k + KO / 2]);
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, t), ors, oo[k], 0, 0);
    }
    return;
  }
  const float* bias2 = a.bias2 ? a.bias2 + (long long)b * a.bias2b : nullptr;
  const float* rb = G.res ? G.res + (long long)b * a.rb : nullptr;
  const __amdgpu_buffer_rsrc_t ors = uniform_rsrc(ob, 4u * (unsigned)((a.C_out - 1) * (int)a.oc + G.n_out));
  float b2v[KO], rv[KO], ov[KO];
  if (bias2) {
    const __amdgpu_buffer_rsrc_t rs = uniform_rsrc(bias2, 4u * (unsigned)a.C_out);
#pragma unroll
    for (int k = 0; k < KO; ++k) b2v[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, bo[k], 0, 0));
  }
  if (rb) {
    const __amdgpu_buffer_rsrc_t rs = uniform_rsrc(rb, 4u * (unsigned)((a.C_out - 1) * (int)a.rc + G.n_out));
#pragma unroll
    for (int k = 0; k < KO; ++k) rv[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, ro[k], 0, 0));
    if (a.res_stat) {
      // the residual's LayerNorm (column statistics from the kernel start)
      const __amdgpu_buffer_rsrc_t gs = uniform_rsrc(a.res_g, 4u * (unsigned)a.C_out);
      const __amdgpu_buffer_rsrc_t bs = uniform_rsrc(a.res_b, 4u * (unsigned)a.C_out);
#pragma unroll
      for (int k = 0; k < KO; ++k) {
        const float g = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(gs, bo[k], 0, 0));
        const float be = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(bs, bo[k], 0, 0));
        rv[k] = (rv[k] - rs_mu) * rs_rd * g + be;
      }
    }
  }
  if (G.combine != COMB_STORE) {
#pragma unroll
    for (int k = 0; k < KO; ++k) ov[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ors, oo[k], 0, 0));
  }
#pragma unroll
  for (int k = 0; k < KO; ++k) {
    float t = v[k];
    if (G.bias) t = t + bv[k];
    if (bias2) t = t + b2v[k];
    if (rb) t = t + rv[k];
    t = apply_act(t, a.out_act, a.out_slope);
    if (G.combine == COMB_ADD) {
      t = ov[k] + t;
    } else if (G.combine == COMB_ADD_DIV) {
      t = (ov[k] + t) / a.div;
    } else if (G.combine == COMB_SUB) {
      t = ov[k] - t;
    }
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, t), ors, oo[k], 0, 0);
    v[k] = t;
  }
  if (a.stat_out) {
    // the next LayerNorm's column statistics of this tile: the 32 stored
    // values of each column through LDS, added in row order by one thread
    __syncthreads();  // every thread has read its partial tiles
#pragma unroll
    for (int k = 0; k < KO; ++k) red[(tid / BN + k * RS) * BN + col] = v[k];
    __syncthreads();
    if (tid < BN && icol) {
      double sm = 0.0, sq = 0.0;
#pragma unroll 8
      for (int r = 0; r < 32; ++r) {
        const double x = red[r * BN + tid];
        sm += x;
        sq += x * x;
      }
      reinterpret_cast<double2*>(a.stat_out)[((long long)b * gridDim.y + blockIdx.y) * G.n_out + i] = make_double2(sm, sq);
    }
  }
}

// 1x1 convs, C_in <= 256: the whole reduction -- x[0:C_in][i0:i0+BN] and
// W[0:C_in][co0:co0+32] -- staged into LDS with one round of loads.
template <int BN>
__global__ __launch_bounds__(256) void conv1x1_small_kernel(ConvLaunch a) {
  constexpr int TN = BN / 32;
  constexpr int RS = 256 / BN;        // input channels one pass of the workgroup stages
  constexpr int LB = 12;              // loads in flight per thread per staging batch
  constexpr unsigned kOut = 0x80000000u;
  extern __shared__ float smem[];
  const int b = blockIdx.z % a.B;
  const int gi = blockIdx.z / a.B;
  const ConvGroup& G = a.g[gi];
  const int i0 = blockIdx.x * BN;
  if (i0 >= G.n_out) return;  // uniform for the whole workgroup, before any barrier
  const int co0 = blockIdx.y * 32;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int C_in = a.C_in;
  // LDS: ws [ceil32(C_in)][32] (rows past C_in zero), then xs
  // [ceil(n_it / LB) * LB * RS][BN] (rows past C_in zero).  Sized to C_in, so
  // a 192-channel reduction at BN = 32 takes 48 KiB and three workgroups fit a
  // CU (enc_p's qkv conv: 576 workgroups in one round, 11.6 -> 9.3 us).
  const int n_it = C_in / RS;  // C_in % 8 == 0, RS <= 8
  float* ws = smem;
  float* xs = smem + ((C_in + 31) & ~31) * 32;

  // the weights (8 float4 loads per thread, rows past C_in read as zero) and
  // the first batch of x in flight together, then the rest of x in batches of
  // LB independent loads: thread tid always stages column tid % BN of rows
  // tid / BN + RS * j, so the bounds test is one comparison per thread.
  const __amdgpu_buffer_rsrc_t wrs = uniform_rsrc(G.w, 4u * (unsigned)(C_in * a.w_ld));
  const __amdgpu_buffer_rsrc_t xrs =
      uniform_rsrc(G.x + (long long)b * a.xb, 4u * (unsigned)((C_in - 1) * (int)a.xc + a.L_in));
  const int cols = (a.C_out + 3) & ~3;
  const int xcol = tid % BN;
  const int xrow = tid / BN;
  const bool xin = i0 + xcol < a.L_in;
  const bool leaky = a.in_act == ACT_LEAKY;
  // kOut + anything below 2^31 stays past the end of the buffer
  const unsigned xbase = xin ? 4u * (unsigned)(xrow * (int)a.xc + i0 + xcol) : kOut;
  const unsigned xstep = 4u * (unsigned)(RS * (int)a.xc);
  auto xload = [&](int j0, float (&v)[LB]) {
#pragma unroll
    for (int j = 0; j < LB; ++j) {
      const unsigned off = j0 + j < n_it ? xbase + (unsigned)(j0 + j) * xstep : kOut;
      v[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xrs, off, 0, 0));
    }
  };
  auto xstore = [&](int j0, const float (&v)[LB]) {
#pragma unroll
    for (int j = 0; j < LB; ++j) {
      float u = v[j];
      if (leaky) u = u >= 0.f ? u : u * a.in_slope;
      xs[(j0 + j) * 256 + tid] = u;
    }
  };
  float4 wv[8];
  {
    const int ci = tid >> 3;
    const int co = co0 + 4 * (tid & 7);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = ci + 32 * j;
      const unsigned off = (c < C_in && co < cols) ? 4u * (unsigned)(c * a.w_ld + co) : kOut;
      wv[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 0, 0));
    }
  }
  // LayerNorm on the way in: gamma / beta go to LDS behind xs, with the
  // column statistics (float64 partial sums [RS][BN], then mean and den)
  const bool ln = a.ln_g != nullptr;
  float* lng = xs + (n_it + LB - 1) / LB * LB * 256;
  float* lnb = lng + 256;
  double* lnp = reinterpret_cast<double*>(lnb + 256);
  float* lnm = reinterpret_cast<float*>(lnp + 256);
  float* lnd = lnm + BN;
  float gv = 0.f, bv0 = 0.f;
  if (ln && tid < C_in) {
    gv = a.ln_g[tid];
    bv0 = a.ln_b[tid];
  }
  for (int j0 = 0; j0 < n_it; j0 += LB) {
    float v[LB];
    xload(j0, v);
    if (j0 == 0) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (32 * j < C_in) reinterpret_cast<float4*>(ws)[tid + 256 * j] = wv[j];  // uniform
      if (ln) {
        lng[tid] = gv;
        lnb[tid] = bv0;
      }
    }
    xstore(j0, v);
  }
  __syncthreads();
  if (ln) {
    // thread (xrow, xcol) staged rows xrow + RS * j, j < n_it, of column xcol.
    // Four float64 accumulators (n_it = C_in / RS is a multiple of 4 for
    // C_in % 8 == 0 and RS <= 8 when C_in % 32 == 0; else the tail loop runs):
    // float64 sums of float32 values this few are exact in any order.
    double s4[4] = {0.0, 0.0, 0.0, 0.0};
    int j = 0;
    for (; j + 4 <= n_it; j += 4)
#pragma unroll
      for (int u = 0; u < 4; ++u) s4[u] += xs[(j + u) * 256 + tid];
    for (; j < n_it; ++j) s4[0] += xs[j * 256 + tid];
    lnp[tid] = (s4[0] + s4[1]) + (s4[2] + s4[3]);
    __syncthreads();
    if (tid < BN) {
      double t = 0.0;
      for (int g = 0; g < RS; ++g) t += lnp[g * BN + tid];
      lnm[tid] = (float)(t / C_in);
    }
    __syncthreads();
    const float mu = lnm[xcol];
    double q4[4] = {0.0, 0.0, 0.0, 0.0};
    j = 0;
    for (; j + 4 <= n_it; j += 4)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float d = xs[(j + u) * 256 + tid] - mu;
        q4[u] += (double)d * d;
      }
    for (; j < n_it; ++j) {
      const float d = xs[j * 256 + tid] - mu;
      q4[0] += (double)d * d;
    }
    lnp[tid] = (q4[0] + q4[1]) + (q4[2] + q4[3]);
    __syncthreads();
    if (tid < BN) {
      double t = 0.0;
      for (int g = 0; g < RS; ++g) t += lnp[g * BN + tid];
      lnd[tid] = 1.0f / sqrtf((float)(t / C_in) + a.ln_eps);
    }
    __syncthreads();
    // every C_out tile of the column block normalises the same staged tile,
    // so the per-element division becomes a multiply by the column's 1 / den
    const float rdn = lnd[xcol];
    const bool wr = blockIdx.y == 0 && a.ln_out != nullptr && i0 + xcol < a.L_in;
    float* lo = a.ln_out + (long long)b * a.ln_ob + i0 + xcol;
#pragma unroll 4
    for (int jj = 0; jj < n_it; ++jj) {
      const int r = xrow + RS * jj;
      const float y = (xs[jj * 256 + tid] - mu) * rdn * lng[r] + lnb[r];
      xs[jj * 256 + tid] = y;
      if (wr) lo[(long long)r * a.ln_oc] = y;
    }
    __syncthreads();
  }

  floatx16 acc[TN];
#pragma unroll
  for (int n = 0; n < TN; ++n)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[n][r] = 0.f;
  // wave w takes input channels [w*q, (w+1)*q), two per MFMA (k = lane / 32)
  const int q = C_in / 4;
  const float* wl = ws + (wave * q + half) * 32 + l32;
  const float* xl = xs + (wave * q + half) * BN + l32;
  int st = 0;
  for (; st + 4 <= q / 2; st += 4) {
    float av[4], bv[4][TN];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      av[u] = wl[2 * (st + u) * 32];
#pragma unroll
      for (int n = 0; n < TN; ++n) bv[u][n] = xl[2 * (st + u) * BN + n * 32];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int n = 0; n < TN; ++n) acc[n] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u], bv[u][n], acc[n], 0, 0, 0);
  }
  for (; st < q / 2; ++st) {
    const float av = wl[2 * st * 32];
#pragma unroll
    for (int n = 0; n < TN; ++n)
      acc[n] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, xl[2 * st * BN + n * 32], acc[n], 0, 0, 0);
  }
  small_conv_epilogue<BN>(a, G, b, i0, co0, false, acc, smem, 0.f, 0.f);
}

// K-tap convs (K = 3, 5 or 7, dilation 1, stride 1), C_in % CHK == 0: the
// reduction streams through LDS in chunks of CHK input channels with all K
// taps -- W[0:K][c0:c0+CHK][32 rows] and x[c0:c0+CHK][i0+in_off : +BN+K-1] --
// the next chunk's loads in flight (registers) while the current one is
// multiplied.  Wave w of NW takes channels [w*CHK/NW, (w+1)*CHK/NW) of every
// chunk, two per MFMA (k = lane / 32), the K taps innermost.  POST_WN_GATE launches
// map tile rows to channel pairs (16 tanh channels and their sigmoid
// partners, cb = blockIdx.y * 16).
template <int BN, int K, int CHK, int NW>
__global__ __launch_bounds__(64 * NW) void conv_small_kernel(ConvLaunch a) {
  constexpr int NT = 64 * NW;
  constexpr int TN = BN / 32;
  constexpr int XW = BN + K - 1;             // staged input columns per channel
  static_assert((K * CHK * 8) % NT == 0 && CHK % (2 * NW) == 0, "whole float4 rows and MFMA steps per wave");
  constexpr int WF4 = K * CHK * 8 / NT;      // float4 weight loads per thread per chunk
  constexpr int XE = (CHK * XW + NT - 1) / NT; // input loads per thread per chunk
  constexpr unsigned kOut = 0x80000000u;
  extern __shared__ float smem[];
  float* ws = smem;                // [K][CHK][32]
  float* xs = smem + K * CHK * 32; // [XE * NT] (CHK rows of XW, tail unused)
  // blockIdx.z = (split * n_groups + group) * B + batch item; sc_split > 1
  // (1x1 launches only): this workgroup reduces over chunks [c_lo, c_hi) of
  // the input channels and stores a raw partial tile
  const int nsplit = a.sc_split > 1 ? a.sc_split : 1;
  const int zb = blockIdx.z % (a.B * a.n_groups);
  const int sidx = blockIdx.z / (a.B * a.n_groups);
  const int b = zb % a.B;
  const int gi = zb / a.B;
  const ConvGroup& G = a.g[gi];
  const int i0 = blockIdx.x * BN;
  if (i0 >= G.n_out) return;  // uniform for the whole workgroup, before any barrier
  const bool gate = a.post == POST_WN_GATE;
  const int co0 = gate ? blockIdx.y * 16 : blockIdx.y * 32;
  const int H = a.post_H;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int C_in = a.C_in;
  const int n_ch = C_in / CHK;
  const int c_lo = sidx * (n_ch / nsplit), c_hi = c_lo + n_ch / nsplit;  // the launcher requires n_ch % nsplit == 0

  const __amdgpu_buffer_rsrc_t wrs = uniform_rsrc(G.w, 4u * (unsigned)(K * C_in * a.w_ld));
  const __amdgpu_buffer_rsrc_t xrs =
      uniform_rsrc(G.x + (long long)b * a.xb, 4u * (unsigned)((C_in - 1) * (int)a.xc + a.L_in));
  // per-thread staging offsets relative to the chunk's first channel
  const int cols = (a.C_out + 3) & ~3;
  unsigned wo[WF4];
#pragma unroll
  for (int j = 0; j < WF4; ++j) {
    const int f = j * NT + tid;  // float4 index in [K][CHK][8]
    const int kc = f >> 3;
    const int k = kc / CHK, ci = kc - k * CHK;
    const int r4 = 4 * (f & 7);
    const int co = gate ? (r4 < 16 ? co0 + r4 : H + co0 + r4 - 16) : co0 + r4;
    wo[j] = co < cols ? 4u * (unsigned)((k * C_in + ci) * a.w_ld + co) : kOut;
  }
  unsigned xo[XE];
#pragma unroll
  for (int j = 0; j < XE; ++j) {
    const int e = j * NT + tid;
    const int ci = e / XW;
    const int t = i0 + G.in_off + (e - ci * XW);
    xo[j] = (e < CHK * XW && t >= 0 && t < a.L_in) ? 4u * (unsigned)(ci * (int)a.xc + t) : kOut;
  }
  float4 wv[WF4];
  float xv[XE];
  auto load = [&](int c) {
    const unsigned wadd = 4u * (unsigned)(c * CHK * a.w_ld);
    const unsigned xadd = 4u * (unsigned)(c * CHK * (int)a.xc);
#pragma unroll
    for (int j = 0; j < WF4; ++j)
      wv[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(wrs, wo[j] == kOut ? kOut : wo[j] + wadd, 0, 0));
#pragma unroll
    for (int j = 0; j < XE; ++j)
      xv[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xrs, xo[j] == kOut ? kOut : xo[j] + xadd, 0, 0));
  };
  const bool leaky = a.in_act == ACT_LEAKY;

  floatx16 acc[TN];
#pragma unroll
  for (int n = 0; n < TN; ++n)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[n][r] = 0.f;
  constexpr int Q = CHK / NW;
  const float* wl = ws + (wave * Q + half) * 32 + l32;
  const float* xl = xs + (wave * Q + half) * XW + l32;
  load(c_lo);
  // LayerNorms from the producers' column statistics (1x1 launches only;
  // a thread stages and finishes one column, tid % BN): of the input while
  // it is staged (no affine: the caller folds gamma / beta into the weights
  // and bias), and of the residual in the epilogue.  xs is free until the
  // first chunk is staged and holds the statistics' scratch.
  constexpr bool kLn = K == 1;
  static_assert(!kLn || (NT % BN == 0 && XE * NT >= 4 * NT + 2 * BN), "a thread stages one column; scratch room");
  const bool ln = kLn && a.ln_stat != nullptr;
  float ln_mu = 0.f, ln_rd = 0.f, rs_mu = 0.f, rs_rd = 0.f;
  if constexpr (kLn) {
    if (ln) ln_column_stats<NT, BN>(a.ln_stat, a.ln_ntile, C_in, a.L_in, a.ln_eps, b, i0, xs, ln_mu, ln_rd);
    if (a.res_stat && nsplit == 1)
      ln_column_stats<NT, BN>(a.res_stat, a.C_out / 32, a.C_out, G.n_out, a.ln_eps, b, i0, xs, rs_mu, rs_rd);
  }
  for (int c = c_lo; c < c_hi; ++c) {
#pragma unroll
    for (int j = 0; j < WF4; ++j) reinterpret_cast<float4*>(ws)[j * NT + tid] = wv[j];
    if (ln) {
#pragma unroll
      for (int j = 0; j < XE; ++j) xs[j * NT + tid] = (xv[j] - ln_mu) * ln_rd;
    } else {
#pragma unroll
      for (int j = 0; j < XE; ++j) {
        float u = xv[j];
        if (leaky) u = u >= 0.f ? u : u * a.in_slope;
        xs[j * NT + tid] = u;
      }
    }
    __syncthreads();
    if (c + 1 < c_hi) load(c + 1);
#pragma unroll 2
    for (int st = 0; st < Q / 2; ++st) {
      float av[K], bv[K][TN];
#pragma unroll
      for (int k = 0; k < K; ++k) {
        av[k] = wl[(k * CHK + 2 * st) * 32];
#pragma unroll
        for (int n = 0; n < TN; ++n) bv[k][n] = xl[2 * st * XW + n * 32 + k];
      }
#pragma unroll
      for (int k = 0; k < K; ++k)
#pragma unroll
        for (int n = 0; n < TN; ++n) acc[n] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[k], bv[k][n], acc[n], 0, 0, 0);
    }
    if (c + 1 < c_hi) __syncthreads();  // the next chunk's stores overwrite this one
  }
  small_conv_epilogue<BN, NW>(a, G, b, i0, co0, gate, acc, smem, rs_mu, rs_rd, nsplit > 1 ? sidx : -1);
}

// The output of a split chunked 1x1 launch (sc_split > 1): for output column
// i of 32-row tile blockIdx.y, out = ((sum_s part[s]) + bias) + res, the
// splits added in index order and the residual normalised from a.res_stat
// when set (the small-conv epilogue's formulas); with a.stat_out, the float64
// (sum, sum of squares) of the tile's stored values per column.  A workgroup
// takes kSrCols columns x the tile's 32 rows, thread (g, c) rows kSrRows * g
// .. + kSrRows - 1 of column c, every operand loaded before the first store;
// the statistics are added per thread in row order, then over g in order.
constexpr int kSrCols = 32, kSrRows = 4, kSrGroups = 256 / kSrCols;  // 384 workgroups at 499 frames
static_assert(kSrGroups * kSrRows == 32, "a workgroup covers the 32 rows of its tile");
__global__ __launch_bounds__(256) void splitk_small_reduce_kernel(ConvLaunch a) {
  const ConvGroup& G = a.g[0];
  const int c = threadIdx.x % kSrCols, rg = threadIdx.x / kSrCols;
  const int i = blockIdx.x * kSrCols + c;
  const int tile = blockIdx.y, b = blockIdx.z;
  const bool icol = i < G.n_out;
  const int S = a.sc_split, ntile = a.C_out / 32;
  __shared__ double red[kSrGroups][kSrCols][2];
  float mu = 0.f, rd = 0.f;
  if (a.res_stat && icol) {
    const double2* st = reinterpret_cast<const double2*>(a.res_stat) + (long long)b * ntile * G.n_out + i;
    double sm = 0.0, sq = 0.0;
    for (int t = 0; t < ntile; ++t) {
      const double2 w = st[(long long)t * G.n_out];
      sm += w.x;
      sq += w.y;
    }
    const double md = sm / a.C_out;
    mu = (float)md;
    rd = 1.0f / sqrtf((float)(fmax(sq - sm * md, 0.0) / a.C_out) + a.ln_eps);
  }
  constexpr unsigned kOut = 0x80000000u;
  const int r0 = tile * 32 + kSrRows * rg;  // this thread's first row
  const unsigned plane = 4u * (unsigned)(a.B * a.C_out * G.n_out);  // bytes of one split's partials
  const __amdgpu_buffer_rsrc_t prs = uniform_rsrc(a.part, plane * (unsigned)S);
  const unsigned po = icol ? 4u * (unsigned)(((long long)b * a.C_out + r0) * G.n_out + i) : kOut;
  const bool hr = G.res != nullptr;
  const __amdgpu_buffer_rsrc_t rrs =
      uniform_rsrc(hr ? G.res + (long long)b * a.rb : G.out, hr ? 4u * (unsigned)(a.C_out * (int)a.rc) : 0u);
  const unsigned ro = icol ? 4u * (unsigned)(r0 * (int)a.rc + i) : kOut;
  float v[kSrRows], rv[kSrRows];
#pragma unroll
  for (int r = 0; r < kSrRows; ++r) {
    v[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(prs, po, 4 * r * G.n_out, 0));
    rv[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rrs, ro, 4 * r * (int)a.rc, 0));
  }
  for (int u = 1; u < S; ++u) {
    const unsigned pu = icol ? po + u * plane : kOut;
#pragma unroll
    for (int r = 0; r < kSrRows; ++r)
      v[r] = v[r] + __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(prs, pu, 4 * r * G.n_out, 0));
  }
  double sm = 0.0, sq = 0.0;
  if (icol) {
    float* op = G.out + (long long)b * a.ob + (long long)r0 * a.oc + i;
#pragma unroll
    for (int r = 0; r < kSrRows; ++r) {
      const int co = r0 + r;
      float t = v[r];
      if (G.bias) t = t + G.bias[co];
      if (hr) {
        float x = rv[r];
        if (a.res_stat) x = (x - mu) * rd * a.res_g[co] + a.res_b[co];
        t = t + x;
      }
      op[(long long)r * a.oc] = t;
      sm += t;
      sq += (double)t * t;
    }
  }
  if (!a.stat_out) return;  // uniform: no barrier follows
  red[rg][c][0] = sm;
  red[rg][c][1] = sq;
  __syncthreads();
  if (rg == 0 && icol) {
    double tsm = red[0][c][0], tsq = red[0][c][1];
    for (int g = 1; g < kSrGroups; ++g) {
      tsm += red[g][c][0];
      tsq += red[g][c][1];
    }
    reinterpret_cast<double2*>(a.stat_out)[((long long)b * ntile + tile) * G.n_out + i] = make_double2(tsm, tsq);
  }
}

// out = combine(act(sum_s part[s] + bias (+ bias2) (+ res))), the splits
// added in index order (deterministic), one thread per output element.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(ConvLaunch a) {
  const ConvGroup& G = a.g[0];
  const long long n = (long long)a.B * a.C_out * G.n_out;
  const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
  if (e >= n) return;
  const int i = (int)(e % G.n_out);
  const int co = (int)((e / G.n_out) % a.C_out);
  const int b = (int)(e / ((long long)G.n_out * a.C_out));
  float v = a.part[e];
  for (int s = 1; s < a.ksplit; ++s) v = v + a.part[e + (long long)s * n];
  if (G.bias) v = v + G.bias[co];
  if (a.bias2) v = v + a.bias2[(long long)b * a.bias2b + co];
  const long long t = (long long)i * G.out_step + G.out_off;
  if (G.res) v = v + G.res[(long long)b * a.rb + (long long)co * a.rc + t];
  v = apply_act(v, a.out_act, a.out_slope);
  float* o = G.out + (long long)b * a.ob + (long long)co * a.oc + t;
  if (G.combine == COMB_ADD) {
    v = *o + v;
  } else if (G.combine == COMB_ADD_DIV) {
    v = (*o + v) / a.div;
  }
  *o = v;
}

// The WaveNet gate of the flow's coupling layers (runtime/models/vits.py:
// 1086-1145) on the split-K sums of the in-layer conv: one thread per (b, c < H, t)
// adds both halves' splits in order, then tanh(a + g_c) * sigmoid(b + g_{H+c})
// in the expression order of the unfused path.
__global__ __launch_bounds__(256) void splitk_reduce_gate_kernel(ConvLaunch a) {
  const ConvGroup& G = a.g[0];
  const int H = a.post_H, L = G.n_out;
  const long long nfull = (long long)a.B * a.C_out * L;
  const long long n = (long long)a.B * H * L;
  const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
  if (e >= n) return;
  const int t = (int)(e % L);
  const int c = (int)((e / L) % H);
  const int b = (int)(e / ((long long)L * H));
  const long long e1 = ((long long)b * a.C_out + c) * L + t;
  const long long e2 = e1 + (long long)H * L;
  float v1 = a.part[e1], v2 = a.part[e2];
  for (int s = 1; s < a.ksplit; ++s) {
    v1 = v1 + a.part[e1 + (long long)s * nfull];
    v2 = v2 + a.part[e2 + (long long)s * nfull];
  }
  if (G.bias) {
    v1 = v1 + G.bias[c];
    v2 = v2 + G.bias[H + c];
  }
  const float* g = a.post_g + (long long)b * a.post_gb;
  G.out[(long long)b * a.ob + (long long)c * a.oc + t] = tanhf(v1 + g[c]) * sigmoid_as(v2 + g[H + c]);
}

// The residual / skip update of a WaveNet layer on the split-K sums of its
// res-skip conv: h[c] += v_c for c < H (not the last layer), the skip
// channels (all of them in the last layer) into skip (= in the first layer).
__global__ __launch_bounds__(256) void splitk_reduce_update_kernel(ConvLaunch a) {
  const ConvGroup& G = a.g[0];
  const int H = a.post_H, L = G.n_out;
  const long long n = (long long)a.B * a.C_out * L;
  const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
  if (e >= n) return;
  const int t = (int)(e % L);
  const int co = (int)((e / L) % a.C_out);
  const int b = (int)(e / ((long long)L * a.C_out));
  float v = a.part[e];
  for (int s = 1; s < a.ksplit; ++s) v = v + a.part[e + (long long)s * n];
  if (G.bias) v = v + G.bias[co];
  const long long hb = ((long long)b * H) * L + t;
  if (!a.post_last && co < H) {
    float* p = a.post_h + hb + (long long)co * L;
    *p = *p + v;
  } else {
    float* p = a.post_skip + hb + (long long)(a.post_last ? co : co - H) * L;
    *p = a.post_first ? v : *p + v;
  }
}

constexpr size_t kLdsLimit = 65536;

int max_n_out(const ConvLaunch& a) {
  int n = 0;
  for (int g = 0; g < a.n_groups; ++g) n = std::max(n, a.g[g].n_out);
  return n;
}

template <int BM, int BN, int WM, int WN, int BK, int SK, int S = 1, int KMAX = kConvTapsMax, int NBUF = 1>
bool launch_cfg(const ConvLaunch& a, hipStream_t s) {
  using C = Cfg<BM, BN, WM, WN, BK, SK, S, KMAX, NBUF>;
  size_t lds = 0;
  for (int g = 0; g < a.n_groups; ++g) lds = std::max(lds, C::lds_bytes(a.g[g].K, a.g[g].dil));
  if (lds > kLdsLimit) return false;
  dim3 grid((max_n_out(a) + BN - 1) / BN, (a.C_out + BM - 1) / BM, a.n_groups * a.B * std::max(a.ksplit, 1));
  for (int g = 0; g < a.n_groups; ++g) RVC_CHECK(a.g[g].K <= KMAX, "conv1d_mfma: taps exceed the configuration");
  hipLaunchKernelGGL((conv1d_mfma_kernel<BM, BN, WM, WN, BK, SK, S, KMAX, NBUF>), grid, dim3(C::NT), lds, s, a);
  check_launch("conv1d_mfma");
  if (a.ksplit > 1) launch_splitk_reduce(a, s);
  return true;
}

// Compute units of the current device (cached per device).
int device_cus() {
  static std::atomic<int> cache[16];
  int dev = 0;
  RVC_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 16) {
    int n = 0;
    RVC_HIP(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
    return n;
  }
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    RVC_HIP(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Workgroups of `kernel` resident per CU with `lds` bytes of dynamic LDS
// (cached per kernel and LDS size: the decoder issues the same few shapes).
int resident_blocks(const void* kernel, int threads, size_t lds) {
  static std::mutex mu;
  static std::map<std::pair<const void*, size_t>, int> cache;
  std::lock_guard<std::mutex> lk(mu);
  auto it = cache.find({kernel, lds});
  if (it != cache.end()) return it->second;
  int nb = 0;
  RVC_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kernel, threads, lds));
  cache[{kernel, lds}] = nb;
  return nb;
}

// The persistent kernel takes stride-1 launches without a channel split, a
// second bias or ADD_DIV, with whole 8-channel chunks, whose groups either
// store (optionally adding a residual) or accumulate without a residual.
bool persist_ok(const ConvLaunch& a) {
  if (a.bias2 || a.ksplit > 1 || a.C_in % 8 != 0) return false;
  // 32-bit byte offsets within one batch item's tensors
  const long long lim = 1LL << 31;
  if (4LL * a.C_out * a.oc >= lim || 4LL * a.C_out * a.rc >= lim || 4LL * a.C_in * a.xc >= lim) return false;
  for (int g = 0; g < a.n_groups; ++g) {
    const ConvGroup& G = a.g[g];
    if (G.K < 1 || G.in_step > 1) return false;
    if (G.combine == COMB_ADD_DIV || (G.combine == COMB_ADD && G.res)) return false;
  }
  return true;
}

template <int BM, int BN, int WM, int WN, int BK, bool DIRECT, int HC>
bool launch_persist_kernel(const ConvLaunch& a, hipStream_t s, int stage, size_t lds, int n_tx, int n_ty, bool fam,
                           long long items) {
  using C = Cfg<BM, BN, WM, WN, BK, 1, 1, kConvTapsMax, 2>;
  const void* k1 = reinterpret_cast<const void*>(&conv1d_mfma_persist_kernel<BM, BN, WM, WN, BK, 1, DIRECT, HC>);
  const void* k0 = reinterpret_cast<const void*>(&conv1d_mfma_persist_kernel<BM, BN, WM, WN, BK, 0, DIRECT, HC>);
  // 64 KiB of staging plus the kernel's static ticket word: allow the
  // dynamic part its full size (a CU holds 160 KiB)
  if (lds > 65536 - 256) {
    static bool attr = false;  // per instantiation
    if (!attr) {
      RVC_HIP(hipFuncSetAttribute(k1, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsLimit));
      RVC_HIP(hipFuncSetAttribute(k0, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsLimit));
      attr = true;
    }
  }
  const int per_cu = resident_blocks(fam ? k1 : k0, C::NT, lds);
  if (per_cu < 1) return false;
  long long grid = (long long)per_cu * device_cus();
  if (grid >= 8) grid -= grid % 8;  // item j then runs on XCD j % 8
  grid = std::min(grid, items);
  const int cpx = device_cus() % 8 == 0 ? device_cus() / 8 : 0;  // CUs per XCD
  if (fam)
    launch_timed(conv1d_mfma_persist_kernel<BM, BN, WM, WN, BK, 1, DIRECT, HC>, dim3((unsigned)grid), dim3(C::NT), lds,
                 s, a, n_tx, n_ty, stage, cpx);
  else
    launch_timed(conv1d_mfma_persist_kernel<BM, BN, WM, WN, BK, 0, DIRECT, HC>, dim3((unsigned)grid), dim3(C::NT), lds,
                 s, a, n_tx, n_ty, stage, cpx);
  check_launch("conv1d_mfma_persist");
  return true;
}

template <int BM, int BN, int WM, int WN, int BK>
bool launch_persist(const ConvLaunch& a, hipStream_t s) {
  if (a.C_out % BM != 0) return false;  // the epilogue has no row guard
  // inputs that take no activation are staged by direct-to-LDS loads
  const bool direct = a.in_act == ACT_NONE;
  // halo class (64-row tiles; the 32-row tiles keep the item's own stride,
  // HC = 0): the staged window's row stride BN + 16 when every group's halo
  // (K - 1) dil fits 16 columns (the dilation-1 launches), else BN + 64
  int halo = 0;
  for (int g = 0; g < a.n_groups; ++g) halo = std::max(halo, (a.g[g].K - 1) * a.g[g].dil);
  const int HC = BM < 64 ? 0 : halo <= 16 ? 16 : kConvHaloMax;
  int stage = 0;  // floats per staging buffer
  if (direct) {
    const int XWC = BN + (HC > 0 ? HC : kConvHaloMax);
    const int xreg = HC > 0 ? (BK * XWC + 63) / 64 * 64 : Cfg<BM, BN, WM, WN, BK, 1, 1, kConvTapsMax, 2>::XPT *
                                                              Cfg<BM, BN, WM, WN, BK, 1, 1, kConvTapsMax, 2>::NT;
    stage = xreg + kConvTapsMax * BK * BM;
  } else {
    for (int g = 0; g < a.n_groups; ++g) {  // the largest group
      const int XW = HC > 0 ? BN + HC : BN + (a.g[g].K - 1) * a.g[g].dil;
      stage = std::max(stage, BK * XW + a.g[g].K * BK * BM);
    }
    stage = (stage + 3) / 4 * 4;  // keeps each buffer's weight block 16-byte aligned
  }
  const size_t lds = 2 * sizeof(float) * (size_t)stage;
  if (lds > kLdsLimit) return false;
  const int n_tx = (max_n_out(a) + BN - 1) / BN;
  const int n_ty = (a.C_out + BM - 1) / BM;
  const long long items = (long long)a.B * n_tx * n_ty * a.n_groups;
  RVC_CHECK(items < (1LL << 30), "conv1d_mfma: launch too large");
  bool fam = a.n_groups == 3;
  for (int g = 0; g < a.n_groups; ++g) fam = fam && a.g[g].combine == COMB_STORE;
  if constexpr (BM < 64) {
    return direct ? launch_persist_kernel<BM, BN, WM, WN, BK, true, 0>(a, s, stage, lds, n_tx, n_ty, fam, items)
                  : launch_persist_kernel<BM, BN, WM, WN, BK, false, 0>(a, s, stage, lds, n_tx, n_ty, fam, items);
  } else {
    if (direct)
      return HC == 16 ? launch_persist_kernel<BM, BN, WM, WN, BK, true, 16>(a, s, stage, lds, n_tx, n_ty, fam, items)
                      : launch_persist_kernel<BM, BN, WM, WN, BK, true, kConvHaloMax>(a, s, stage, lds, n_tx, n_ty,
                                                                                     fam, items);
    return HC == 16 ? launch_persist_kernel<BM, BN, WM, WN, BK, false, 16>(a, s, stage, lds, n_tx, n_ty, fam, items)
                    : launch_persist_kernel<BM, BN, WM, WN, BK, false, kConvHaloMax>(a, s, stage, lds, n_tx, n_ty,
                                                                                    fam, items);
  }
}

// Split-K plan for a single-group stride-1 launch whose output tiles alone
// cannot fill the GPU: 128 x 128 (or 64 x 128) tiles and the input channels
// cut into S splits of whole BKT-channel chunks (at least two chunks each),
// so tiles x S reaches about 384 workgroups.  Depends on the per-item tile
// count only, never on B, so batched calls keep the per-chunk results.
long long n_blocks(const ConvLaunch& a, int BM, int BN);

struct SplitPlan {
  int S = 1, csplit = 0, BM = 0;
};
// The small 1x1 GEMM path: every group a plain 1x1 conv (no stride, offset or
// output interleave), at most 256 input channels (the whole reduction fits
// LDS), a few thousand columns, no reduce post-op.
// 32-bit buffer offsets of the small-conv kernels: x, the weights, out and
// the residual each within 2 GiB of their batch item; grid z in range.
bool small_offsets_ok(const ConvLaunch& a) {
  const long long n_out = max_n_out(a);
  return (long long)a.n_groups * a.B <= 65535 && 4LL * ((a.C_in - 1) * a.xc + a.L_in) < (1LL << 31) &&
         4LL * a.g[0].K * a.C_in * a.w_ld < (1LL << 31) && 4LL * ((a.C_out - 1) * a.oc + n_out) < (1LL << 31) &&
         4LL * ((a.C_out - 1) * a.rc + n_out) < (1LL << 31);
}

bool small_gemm_ok(const ConvLaunch& a) {
  if (a.C_in > 256 || a.C_in % 8 != 0 || a.post != POST_NONE || !small_offsets_ok(a)) return false;
  for (int g = 0; g < a.n_groups; ++g) {
    const ConvGroup& G = a.g[g];
    if (G.K != 1 || G.in_step > 1 || G.in_off != 0 || G.out_step != 1 || G.out_off != 0 || G.n_out > 8192 ||
        G.n_out > a.L_in)
      return false;
  }
  return true;
}

// The chunked path: K = 3, 5 or 7 at dilation 1 in every group (C_in a
// multiple of 64 up to 1024), or 1x1 GEMMs too wide for the whole-reduction kernel
// (C_in a multiple of 128 up to 4096); stride 1, a few thousand columns and a
// tile grid too small to fill the GPU (where the split-K path would run); the
// reduce post-op POST_WN_GATE when C_out = 2 * post_H with post_H % 16 == 0.
bool small_conv_ok(const ConvLaunch& a) {
  const int K = a.g[0].K;
  if (K == 1 ? (a.C_in % 128 != 0 || a.C_in > 4096) : (a.C_in % 64 != 0 || a.C_in > 1024)) return false;
  if (!small_offsets_ok(a)) return false;
  if (a.post == POST_WN_GATE) {
    if (a.n_groups != 1 || a.post_H % 16 != 0 || a.C_out != 2 * a.post_H) return false;
  } else if (a.post != POST_NONE) {
    return false;
  }
  if (K != 1 && K != 3 && K != 5 && K != 7) return false;
  for (int g = 0; g < a.n_groups; ++g) {
    const ConvGroup& G = a.g[g];
    if (G.K != K || G.dil != 1 || G.in_step > 1 || G.out_step != 1 || G.out_off != 0 || G.n_out > 8192 ||
        G.in_off > 0 || G.in_off < -(K - 1))
      return false;
  }
  return n_blocks(a, 64, 128) < 384;
}

// The reduction split of a chunked 1x1 launch, a function of the shape only
// (so a batch and its items take the same summation order): the long
// reductions (C_in >= 3072: HuBERT's FFN output GEMM, 384 workgroups of 24
// chunks at 499 frames) run as two splits (768 workgroups of 12 chunks, three
// per CU), their raw partial tiles through part, and
// splitk_small_reduce_kernel forms the output.  Plain epilogues only: bias,
// a residual (LayerNorm'ed from statistics or not), column statistics out.
int small_conv_split(const ConvLaunch& a) {
  if (a.n_groups != 1 || a.g[0].K != 1 || a.C_in < 3072 || a.C_in % 256 != 0 || a.C_out % 32 != 0) return 1;
  if (a.post != POST_NONE || a.out_act != ACT_NONE || a.in_act != ACT_NONE || a.bias2 || a.ln_stat || a.ln_g)
    return 1;
  if (a.g[0].combine != COMB_STORE || a.g[0].in_step > 1 || small_gemm_ok(a) || !small_conv_ok(a)) return 1;
  return 2;
}

template <int BN, int K, int CHK, int NW>
void launch_small_conv_cfg(const ConvLaunch& a, dim3 grid, hipStream_t s) {
  constexpr int NT = 64 * NW;
  constexpr int XE = (CHK * (BN + K - 1) + NT - 1) / NT;
  constexpr size_t lds_stage = sizeof(float) * ((size_t)K * CHK * 32 + (size_t)XE * NT);
  constexpr size_t lds_red = sizeof(float) * NW * (BN / 32) * 16 * 64;  // the epilogue's partial tiles
  static_assert((lds_stage > lds_red ? lds_stage : lds_red) <= 160 * 1024, "staging LDS above the CU's 160 KiB");
  RVC_CHECK((!a.ln_stat || a.ln_ntile <= 4 * (NT / BN)) && (!a.res_stat || a.C_out / 32 <= 4 * (NT / BN)),
            "conv_small: too many statistics tiles for a staged LayerNorm");
  constexpr size_t lds = lds_stage > lds_red ? lds_stage : lds_red;
  // the gate epilogue pairs tile rows k and k + KO / 2 of one thread
  RVC_CHECK(a.post != POST_WN_GATE || 32 * BN / (64 * NW) >= 2,
            "conv_small: the WaveNet gate needs at least two tile rows per thread");
  if (lds > 65536) {
    static bool attr = false;  // per instantiation
    if (!attr) {
      RVC_HIP(hipFuncSetAttribute((const void*)conv_small_kernel<BN, K, CHK, NW>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
      attr = true;
    }
  }
  launch_timed(conv_small_kernel<BN, K, CHK, NW>, grid, dim3(NT), lds, s, a);
}

bool launch_small_conv(const ConvLaunch& a, hipStream_t s) {
  const int n_out = max_n_out(a);
  const bool gate = a.post == POST_WN_GATE;
  RVC_CHECK(!gate || a.post_g, "conv1d_mfma: the WaveNet gate needs its conditioning vector");
  const int nco = gate ? a.post_H / 16 : (a.C_out + 31) / 32;
  const long long z = (long long)a.n_groups * a.B;
  const int K = a.g[0].K;
  // 64-column tiles when they give at least 320 workgroups, else 32: below
  // that, twice the workgroups (two waves per SIMD on more CUs) beat the wider
  // tile's operand reuse (config 2: flow 0.375 -> 0.360 ms, enc_p 0.725 ->
  // 0.709 ms against a threshold of 192).  The reduction order does not
  // depend on the tile width or the batch.
  // The tall 1x1 GEMMs (C_out >= 2304: HuBERT's q/k/v and FFN input) and
  // the short-reduction 3-tap convs (enc_p's FFN input, C_in 192) stay on 32
  // columns: 1152 / 1536 / 768 workgroups instead of 576 / 768 / 384 even out
  // the per-CU load (config 3 3400 -> 3490 audio-s/s, q/k/v 0.453 -> 0.391 ms;
  // enc_p 0.63 -> 0.61 ms).
  const bool wide = (long long)((n_out + 63) / 64) * nco * z >= 320 && !(K == 1 && a.C_out >= 2304) &&
                    !(K == 3 && a.C_in < 512);
  const int BN = wide ? 64 : 32;
  // 128-channel chunks for the long 3-tap reductions (enc_p's FFN output
  // conv, C_in = 768): half the chunk round trips.  Never for a gated launch:
  // those run on sixteen waves, whose 32-column epilogue gives each thread a
  // single tile row, and the gate pairs rows k and k + KO / 2 of one thread.
  const int CHK = K == 3 && a.C_in % 128 == 0 && a.C_in >= 512 && !gate ? 128 : 64;
  const dim3 grid((unsigned)((n_out + BN - 1) / BN), (unsigned)nco, (unsigned)z);
  // Waves per workgroup (each taking its share of every chunk's channels):
  // sixteen for the 128-channel 3-tap chunks (enc_p's FFN output conv, 768 x
  // 3), eight for the other K-tap convs and the 1x1 GEMMs.  Measured at
  // config 2 against four waves: FFN output conv 24.6 -> 20.6 us (8) -> 18.8
  // us (16), WaveNet in-layer 18.2 -> 16.7 us, FFN input conv 19.3 -> 17.8 us;
  // at config 3 the 32-column 1x1 GEMMs (out-proj, FFN output) 35.2 -> 32.3 us
  // (8) / 31.0 us (16, but the 64-column ones 39 -> 43 us).  A function of the
  // shape only, never of B or the tile width (which depends on B): the wave
  // count sets the summation order.
  if (K == 1) {
    const int ss = small_conv_split(a);
    if (ss > 1 && a.part && a.part_floats >= (size_t)ss * a.B * a.C_out * n_out &&
        4.0 * ss * a.B * a.C_out * n_out < 2147483648.0) {
      ConvLaunch sa = a;
      sa.sc_split = ss;
      const dim3 gs(grid.x, grid.y, grid.z * (unsigned)ss);
      wide ? launch_small_conv_cfg<64, 1, 128, 8>(sa, gs, s) : launch_small_conv_cfg<32, 1, 128, 8>(sa, gs, s);
      check_launch("conv_small");
      launch_timed(splitk_small_reduce_kernel, dim3((unsigned)((n_out + kSrCols - 1) / kSrCols), (unsigned)(a.C_out / 32), (unsigned)a.B),
                   dim3(256), 0, s, sa);
      check_launch("conv_small reduce");
      return true;
    }
    wide ? launch_small_conv_cfg<64, 1, 128, 8>(a, grid, s) : launch_small_conv_cfg<32, 1, 128, 8>(a, grid, s);
  } else if (K == 3) {
    if (CHK == 128)
      wide ? launch_small_conv_cfg<64, 3, 128, 16>(a, grid, s) : launch_small_conv_cfg<32, 3, 128, 16>(a, grid, s);
    else
      wide ? launch_small_conv_cfg<64, 3, 64, 8>(a, grid, s) : launch_small_conv_cfg<32, 3, 64, 8>(a, grid, s);
  } else if (K == 5) {
    wide ? launch_small_conv_cfg<64, 5, 64, 8>(a, grid, s) : launch_small_conv_cfg<32, 5, 64, 8>(a, grid, s);
  } else {
    wide ? launch_small_conv_cfg<64, 7, 64, 8>(a, grid, s) : launch_small_conv_cfg<32, 7, 64, 8>(a, grid, s);
  }
  check_launch("conv_small");
  return true;
}

bool launch_small_gemm(const ConvLaunch& a, hipStream_t s) {
  int n_out = 0;
  for (int g = 0; g < a.n_groups; ++g) n_out = std::max(n_out, a.g[g].n_out);
  const int nco = (a.C_out + 31) / 32;
  const long long z = (long long)a.n_groups * a.B;
  const bool wide = (long long)((n_out + 63) / 64) * nco * z >= 320;  // as in launch_small_conv
  const int BN = wide ? 64 : 32;
  // ws: C_in rounded up to 32 rows of 32; xs: the staging passes rounded up
  // to the batch of 12, 256 floats each; the epilogue's four waves' tiles
  const size_t n_it = (size_t)a.C_in / (256 / BN);
  // the LayerNorm's gamma / beta (256 each), float64 partials (256) and the
  // mean / den columns (BN each) behind xs
  const size_t ln_floats = a.ln_g ? 256 + 256 + 2 * 256 + 2 * 64 : 0;
  const size_t lds =
      sizeof(float) * std::max(((size_t)a.C_in + 31) / 32 * 32 * 32 + (n_it + 11) / 12 * 12 * 256 + ln_floats,
                               (size_t)4 * (BN / 32) * 1024);
  constexpr int kMaxLds = sizeof(float) * (256 * 32 + 72 * 256 + 1152);  // C_in = 256, BN = 64, LayerNorm
  RVC_CHECK(!a.ln_g || (a.n_groups == 1 && a.in_act == ACT_NONE && a.ln_b),
            "conv1x1_small: the staged LayerNorm takes one group, no input activation, gamma and beta");
  RVC_CHECK(lds <= (size_t)kMaxLds, "conv1x1_small: LDS above its limit");
  const dim3 grid((unsigned)((n_out + BN - 1) / BN), (unsigned)nco, (unsigned)z);
  static bool attr = false;
  if (!attr) {
    RVC_HIP(hipFuncSetAttribute((const void*)conv1x1_small_kernel<64>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                kMaxLds));
    RVC_HIP(hipFuncSetAttribute((const void*)conv1x1_small_kernel<32>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                kMaxLds));
    attr = true;
  }
  if (wide)
    launch_timed(conv1x1_small_kernel<64>, grid, dim3(256), lds, s, a);
  else
    launch_timed(conv1x1_small_kernel<32>, grid, dim3(256), lds, s, a);
  check_launch("conv1x1_small");
  return true;
}

SplitPlan split_plan(const ConvLaunch& a) {
  SplitPlan p;
  if (a.n_groups != 1 || (a.g[0].in_step > 1) || a.g[0].K < 1) return p;
  if (small_gemm_ok(a) || small_conv_ok(a)) return p;  // no split: a small-conv kernel takes the whole reduction
  const bool gemm = a.g[0].K == 1;
  int BM = 0, BKT = 0;
  if (a.C_out % 128 == 0) {
    BM = 128;
    BKT = gemm ? 32 : 8;
  } else if (a.C_out % 64 == 0) {
    BM = 64;
    BKT = gemm ? 32 : 16;
  } else {
    return p;
  }
  if (n_blocks(a, 64, 128) >= 384) return p;  // the tile grid alone fills the GPU
  const long long nb = n_blocks(a, BM, 128);
  const int max_s = a.C_in / (2 * BKT);
  // about 384 workgroups: measured against 256 / 320 / 448 / 640 on the
  // enc_p + flow convs (P = 1000) and HuBERT's 499-frame GEMMs, where more
  // splits cost more in partial-sum traffic than they gain in parallelism
  int S = (int)std::min<long long>((384 + nb - 1) / nb, max_s);
  if (S < 2) return p;
  const int chunks = (a.C_in + BKT - 1) / BKT;
  const int per = (chunks + S - 1) / S;
  p.csplit = per * BKT;
  p.S = (a.C_in + p.csplit - 1) / p.csplit;
  p.BM = BM;
  return p;
}

// Workgroups per batch item.  The tile choice deliberately ignores B: the
// reduction order depends on the tile, so a batched call stays bit-identical
// to the same chunks run one by one.
long long n_blocks(const ConvLaunch& a, int BM, int BN) {
  long long n = 0;
  for (int g = 0; g < a.n_groups; ++g) n += (long long)((a.g[g].n_out + BN - 1) / BN) * ((a.C_out + BM - 1) / BM);
  return n;
}

}  // namespace

void launch_splitk_reduce(const ConvLaunch& a, hipStream_t s) {
  const long long n = (long long)a.B * a.C_out * a.g[0].n_out;
  if (n <= 0) return;
  if (a.post == POST_WN_GATE) {
    const long long ng = (long long)a.B * a.post_H * a.g[0].n_out;
    hipLaunchKernelGGL(splitk_reduce_gate_kernel, dim3((unsigned)((ng + 255) / 256)), dim3(256), 0, s, a);
  } else if (a.post == POST_WN_UPDATE) {
    hipLaunchKernelGGL(splitk_reduce_update_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a);
  }
  check_launch("splitk_reduce");
}

bool conv1d_mfma_small_path(const ConvLaunch& a) {
  return a.g[0].in_step <= 1 && (small_gemm_ok(a) || small_conv_ok(a));
}

bool conv1d_mfma_fuses_gate(const ConvLaunch& a) {
  ConvLaunch t = a;
  t.post = POST_WN_GATE;
  t.post_H = a.C_out / 2;
  return (a.C_out % 2 == 0 && small_conv_ok(t)) || split_plan(t).S > 1;
}

size_t conv1d_mfma_split_floats(const ConvLaunch& a) {
  const int ss = small_conv_split(a);
  if (ss > 1) return (size_t)ss * a.B * a.C_out * a.g[0].n_out;
  const SplitPlan p = split_plan(a);
  return p.S > 1 ? (size_t)p.S * a.B * a.C_out * a.g[0].n_out : 0;
}

bool conv1d_mfma_supported(int K, int dil) {
  return K >= 0 && K <= kConvTapsMax && dil >= 1 && (K > 0 ? (K - 1) * dil : 0) <= kConvHaloMax;
}

bool conv1d_mfma_chunked_1x1(const ConvLaunch& a) {
  return a.n_groups == 1 && a.g[0].K == 1 && (a.g[0].in_step <= 1) && a.post == POST_NONE && !small_gemm_ok(a) &&
         small_conv_ok(a);
}

void launch_conv1d_mfma(const ConvLaunch& a, hipStream_t s) {
  RVC_CHECK(a.n_groups >= 1 && a.n_groups <= kMaxConvGroups, "conv1d_mfma: bad group count");
  RVC_CHECK(a.C_in >= 1 && a.C_out >= 1 && a.B >= 1 && a.w_ld >= a.C_out && a.w_ld % 4 == 0,
            "conv1d_mfma: invalid shape");
  const int step = a.g[0].in_step <= 1 ? 1 : a.g[0].in_step;
  RVC_CHECK(step == 1 || step == 2, "conv1d_mfma: input stride must be 1 or 2");
  RVC_CHECK(a.post == POST_NONE || (a.n_groups == 1 && step == 1 && (a.part || small_conv_ok(a))),
            "conv1d_mfma: a reduce post-op needs the split-K or the small-conv path");
  for (int g = 0; g < a.n_groups; ++g) {
    RVC_CHECK(a.g[g].n_out >= 0 && conv1d_mfma_supported(a.g[g].K, a.g[g].dil),
              "conv1d_mfma: taps / dilation outside the MFMA path");
    RVC_CHECK((a.g[g].in_step <= 1 ? 1 : a.g[g].in_step) == step, "conv1d_mfma: groups must share the input stride");
    RVC_CHECK((reinterpret_cast<uintptr_t>(a.g[g].w) & 15) == 0, "conv1d_mfma: weights must be 16-byte aligned");
  }
  if (max_n_out(a) == 0) return;
  if (a.ln_stat) {
    RVC_CHECK(conv1d_mfma_chunked_1x1(a) && a.in_act == ACT_NONE && a.ln_ntile >= 1 && a.ln_ntile * 32 == a.C_in,
              "conv1d_mfma: a LayerNorm from producer statistics needs the chunked 1x1 kernel (one group, no input "
              "activation, C_in / 32 statistics tiles)");
  } else {
    RVC_CHECK(!a.ln_g || (step == 1 && small_gemm_ok(a)),
              "conv1d_mfma: a staged LayerNorm needs the whole-reduction 1x1 kernel (C_in <= 256, <= 8192 columns)");
  }
  RVC_CHECK(!a.stat_out || (step == 1 && a.n_groups == 1 && a.C_out % 32 == 0 && a.post == POST_NONE &&
                            (small_gemm_ok(a) || small_conv_ok(a))),
            "conv1d_mfma: column statistics need a small-conv kernel (one group, C_out % 32 == 0)");
  RVC_CHECK(!a.res_stat || (conv1d_mfma_chunked_1x1(a) && a.C_out % 32 == 0 && a.g[0].res && a.res_g && a.res_b),
            "conv1d_mfma: a residual LayerNorm needs the chunked 1x1 kernel, a residual, gamma and beta");
  if (step == 1 && small_gemm_ok(a) && launch_small_gemm(a, s)) return;
  if (step == 1 && small_conv_ok(a) && launch_small_conv(a, s)) return;
  for (int g = 0; g < a.n_groups; ++g)
    RVC_CHECK(a.g[g].combine != COMB_SUB, "conv1d_mfma: the subtracting combine runs on the small-conv kernels only");
  // Tile choice: widest co tile that divides C_out while the grid still
  // gives every CU work (256 CUs); few output columns -> split-K waves.
  // The 128 x 128 tile (two resident workgroups per CU) also needs about two
  // rounds of workgroups, or the longest-tap groups of a grouped launch set
  // the makespan (measured: the C = 256 decoder stage runs 10 % faster on
  // 64 x 128 tiles).
  const long long want = 384;
  bool ok = false;
  if (step == 2) {
    // strided convolutions (the HuBERT feature extractor)
    // KMAX = 3 when every group has at most 3 taps (HuBERT's k3 / k2): the
    // weight prefetch takes 3 taps of registers instead of 11, and the
    // feature-extractor convs run 9-12 % faster (conv1 347 -> 305 us)
    int kmax = 0;
    for (int g = 0; g < a.n_groups; ++g) kmax = std::max(kmax, a.g[g].K);
    if (kmax <= 3) {
      // 128 x 128 where it still gives two rounds of tiles (HuBERT's first
      // stride-2 conv: 310 -> 287 us against 64 x 128)
      if (a.C_out % 128 == 0 && n_blocks(a, 128, 128) >= want) ok = launch_cfg<128, 128, 64, 64, 16, 1, 2, 3>(a, s);
      if (!ok && a.C_out % 64 == 0 && n_blocks(a, 64, 128) >= want) ok = launch_cfg<64, 128, 32, 64, 16, 1, 2, 3>(a, s);
      if (!ok && a.C_out % 64 == 0 && n_blocks(a, 64, 64) >= want) ok = launch_cfg<64, 64, 32, 32, 16, 1, 2, 3>(a, s);
      if (!ok) ok = launch_cfg<32, 64, 32, 32, 8, 4, 2, 3>(a, s);
    }
    if (!ok && a.C_out % 64 == 0 && n_blocks(a, 64, 128) >= want)
      ok = launch_cfg<64, 128, 32, 64, 16, 1, 2>(a, s) || launch_cfg<64, 128, 32, 64, 8, 1, 2>(a, s);
    if (!ok && a.C_out % 64 == 0 && n_blocks(a, 64, 64) >= want) ok = launch_cfg<64, 64, 32, 32, 16, 1, 2>(a, s);
    if (!ok) ok = launch_cfg<32, 64, 32, 32, 8, 4, 2>(a, s) || launch_cfg<32, 64, 32, 32, 4, 4, 2>(a, s);
    RVC_CHECK(ok, "conv1d_mfma: no tile configuration fits the LDS budget");
    return;
  }
  if (a.part && a.part_floats > 0) {
    const SplitPlan p = split_plan(a);
    if (p.S > 1 && (size_t)p.S * a.B * a.C_out * a.g[0].n_out <= a.part_floats) {
      ConvLaunch sa = a;
      sa.ksplit = p.S;
      sa.csplit = p.csplit;
      if (a.g[0].K == 1)
        ok = p.BM == 128 ? launch_cfg<128, 128, 64, 64, 32, 1, 1, 1>(sa, s) : launch_cfg<64, 128, 32, 64, 32, 1, 1, 1>(sa, s);
      else
        ok = p.BM == 128 ? launch_cfg<128, 128, 64, 64, 8, 1>(sa, s) : launch_cfg<64, 128, 32, 64, 16, 1>(sa, s);
      if (ok) return;
    }
  }
  RVC_CHECK(a.post == POST_NONE, "conv1d_mfma: a reduce post-op needs the split-K or the small-conv path");
  int kmax = 0;
  for (int g = 0; g < a.n_groups; ++g) kmax = std::max(kmax, a.g[g].K);
  if (kmax == 1) {  // 1x1 convolutions: plain GEMMs with 32-channel chunks
    if (a.C_out % 128 == 0 && n_blocks(a, 128, 128) >= want) ok = launch_cfg<128, 128, 64, 64, 32, 1, 1, 1>(a, s);
    if (!ok && a.C_out % 64 == 0 && n_blocks(a, 64, 128) >= want) ok = launch_cfg<64, 128, 32, 64, 32, 1, 1, 1>(a, s);
    if (ok) return;
  }
  // Large grids (decoder stages 1-3): 8-wave 64x256 / 32x512 tiles of 32x64
  // wave tiles, which keep the registers near 90 per lane, so five waves per
  // SIMD hide the staging and barrier phases of one another.
  const bool persist = persist_ok(a);
  if (a.C_out % 64 == 0 && n_blocks(a, 64, 256) >= 900)
    ok = (persist && launch_persist<64, 256, 32, 64, 8>(a, s)) || launch_cfg<64, 256, 32, 64, 8, 1>(a, s);
  // The persistent 64 x 256 tile also where its 300 .. 2 x CUs tiles per
  // batch item fit one round of its slots (two per CU; decoder stage 0, C =
  // 256: 480 tiles at 40k / P = 1000, 348 at 48k / P = 600): each input window
  // is staged for 64 output rows instead of 32.  Against the 32 x 256
  // persistent tile (P = 1000) stage 0 went 1.50-1.52 -> 1.42-1.44 ms, config
  // 2 1108-1112 -> 1116-1119 audio-s/s; against the one-shot 64 x 128 tile
  // that takes stage 0 below 900 32 x 256 tiles, config 4 (B = 8) 1097 ->
  // 1115-1119 audio-s/s, but a single P = 700 call 6.98 -> 7.10 ms (336 items
  // fill two thirds of the slots).  The choice may not depend on B (the
  // one-shot tile sums in another order), so the window follows the benchmark
  // shapes.  Between one and two rounds the 32 x 256 items balance better
  // (P = 380: stages 1-2 with 891-894 tiles, 4.30 against 4.60 ms per call).
  if (!ok && persist && a.C_out % 64 == 0) {
    const long long nb = n_blocks(a, 64, 256);
    if (nb >= 300 && nb <= 2LL * device_cus()) ok = launch_persist<64, 256, 32, 64, 8>(a, s);
  }
  if (!ok && a.C_out <= 32 && n_blocks(a, 32, 512) >= 900)
    ok = (persist && launch_persist<32, 512, 32, 64, 8>(a, s)) || launch_cfg<32, 512, 32, 64, 8, 1>(a, s);
  // shorter grids still (stage 0 of short chunks, under 300 tiles of 64 x
  // 256): four-wave 32 x 256 persistent tiles, twice the items (measured 94
  // vs 91 TFLOP/s for the 64 x 128 one-shot tile on C = 256 ResBlock launches)
  if (!ok && persist && a.C_out % 32 == 0 && n_blocks(a, 32, 256) >= 900)
    ok = launch_persist<32, 256, 32, 64, 8>(a, s);
  if (!ok && a.C_out % 128 == 0 && n_blocks(a, 128, 128) >= 900) ok = launch_cfg<128, 128, 64, 64, 8, 1>(a, s);
  if (!ok && a.C_out % 64 == 0 && n_blocks(a, 64, 128) >= want)
    ok = launch_cfg<64, 128, 32, 64, 8, 1>(a, s) || launch_cfg<64, 128, 32, 64, 16, 1>(a, s);
  if (!ok && a.C_out <= 32 && n_blocks(a, 32, 256) >= want)
    ok = launch_cfg<32, 256, 32, 64, 16, 1>(a, s) || launch_cfg<32, 256, 32, 64, 8, 1>(a, s);
  if (!ok && a.C_out % 64 == 0 && n_blocks(a, 64, 64) >= want)
    ok = launch_cfg<64, 64, 32, 32, 16, 1>(a, s) || launch_cfg<64, 64, 32, 32, 8, 1>(a, s);
  if (!ok) ok = launch_cfg<32, 64, 32, 32, 8, 4>(a, s) || launch_cfg<32, 64, 32, 32, 4, 4>(a, s);
  RVC_CHECK(ok, "conv1d_mfma: no tile configuration fits the LDS budget");
}

}  // namespace rvc
