// Implicit-GEMM conv1d on CDNA4 bf16 matrix cores (v_mfma_f32_32x32x16_bf16),
// fp32 accumulate: the bf16 variant of conv_mfma.hip for the mixed-precision
// synthesis modes (the GeneratorNSF upsample convs and the
// enc_p matmuls; optionally the decoder ResBlocks).
//
//   out[b][co][i] = sum_{ci,k} bf16(W[co][ci][k]) * bf16(act(x[b][ci][i + in_off + k*dil]))
//
// with the products summed in fp32.  Same launch description (ConvLaunch,
// grouped grids, polyphase output index i*out_step + out_off, accumulator
// start from bias / residual / accumulate target, split-K partials reduced by
// splitk_reduce_kernel) as the fp32 kernel; input stride 1 only.
//
// The MFMA consumes 16 reduction indices per step; lane l supplies 8 of them
// (k-slots 8*(l/32)..+8) for row l%32 of A and column l%32 of B, and only the
// pairing of A's and B's slots matters, so the 16 slots are 16 consecutive
// input channels.  LDS therefore holds both operands channel-contiguous:
//   xs[pos][ci]      (the input window, bf16, row stride BKT+8)
//   ws[k][co][ci]    (the chunk's weights of every tap, bf16, row stride BKT+8)
// and each operand fragment is one 16-byte LDS read; the +8 padding makes the
// 16 lanes of a read quarter hit 16 distinct 4-bank groups.  The input is
// converted to bf16 (round to nearest even) while it is staged, after the
// optional leaky ReLU; the weights arrive packed in bf16 as [K][C_out][w16_ld].
#include <algorithm>

#include "internal.h"

namespace rvc {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

namespace {

__device__ __forceinline__ float act_b(float v, int act, float slope) {
  if (act == ACT_LEAKY) return v >= 0.f ? v : v * slope;
  if (act == ACT_TANH) return tanhf(v);
  if (act == ACT_RELU) return fmaxf(v, 0.f);
  if (act == ACT_GELU) return gelu_as(v);
  return v;
}

// two floats -> two bf16 (round to nearest even) in one 32-bit word, lo first
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  uint32_t a = __float_as_uint(lo), b = __float_as_uint(hi);
  a += 0x7fffu + ((a >> 16) & 1u);
  b += 0x7fffu + ((b >> 16) & 1u);
  return (a >> 16) | (b & 0xffff0000u);
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) {
  bf16x8 r;
  __builtin_memcpy(&r, &v, 16);
  return r;
}

template <int BM, int BN, int WM, int WN, int BKT, int KMAX>
struct CfgB {
  static constexpr int NWM = BM / WM;
  static constexpr int NWN = BN / WN;
  static constexpr int NT = NWM * NWN * 64;
  static constexpr int TM = WM / 32;
  static constexpr int TN = WN / 32;
  static constexpr int RS = BKT + 8;  // LDS row stride in bf16
  static constexpr int XWMAX = BN + (KMAX > 1 ? kConvHaloMax : 0);
  static constexpr int XPT = ((BKT / 2) * XWMAX + NT - 1) / NT;    // channel pairs per thread
  static constexpr int WV = BKT / 8;                                // 16-byte vectors per weight row
  static constexpr int WPT = (KMAX * BM * WV + NT - 1) / NT;
  static size_t lds_bytes(int K, int dil) {
    const int XW = BN + (K > 0 ? (K - 1) * dil : 0);
    return 2 * ((size_t)XW * RS + (size_t)K * BM * RS);
  }
};

template <int BM, int BN, int WM, int WN, int BKT, int KMAX>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64)
__attribute__((amdgpu_waves_per_eu(2)))
void conv1d_bf16_kernel(ConvLaunch a) {
  using C = CfgB<BM, BN, WM, WN, BKT, KMAX>;
  constexpr int NT = C::NT, TM = C::TM, TN = C::TN, RS = C::RS, XPT = C::XPT, WPT = C::WPT, WV = C::WV;
  static_assert(BKT % 16 == 0, "channel chunk must be a multiple of 16");

  const int b = blockIdx.z % a.B;
  const int gi = (blockIdx.z / a.B) % a.n_groups;
  const int ks = blockIdx.z / (a.B * a.n_groups);
  const ConvGroup& G = a.g[gi];
  const int i0 = blockIdx.x * BN;
  const int csplit = a.ksplit > 1 ? a.csplit : a.C_in;
  const int ci_lo = ks * csplit;
  const int ci_hi = min(a.C_in, ci_lo + csplit);
  if (i0 >= G.n_out) return;  // uniform for the workgroup, before any barrier
  const int co0 = blockIdx.y * BM;
  const int K = G.K;
  const int dil = G.dil;
  const int XW = BN + (K > 0 ? (K - 1) * dil : 0);

  extern __shared__ __attribute__((aligned(16))) uint16_t smem16[];
  uint16_t* xs = smem16;            // [XW][RS]
  uint16_t* ws = smem16 + XW * RS;  // [K][BM][RS]   (XW*RS*2 is a multiple of 16 bytes)

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % C::NWM;
  const int wn = wave / C::NWM;
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

  // accumulator start: bias (+ bias2) (+ residual) (+ the output of an
  // accumulating launch without activation); split-K partials stay raw
  const bool fold_out = G.combine == COMB_ADD && a.out_act == ACT_NONE;
  const float* bias2 = a.bias2 ? a.bias2 + (long long)b * a.bias2b : nullptr;
  float* ob = G.out + (long long)b * a.ob;
  const float* rb = G.res ? G.res + (long long)b * a.rb : nullptr;
  if (a.ksplit <= 1) {
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

  float2 xr[XPT];
  uint4 wreg[WPT];
  const int npair = (BKT / 2) * XW;
  const int nwv = K * BM * WV;
  const int tbase = i0 + G.in_off;

  auto gload = [&](int ci0) {
#pragma unroll
    for (int e = 0; e < XPT; ++e) {
      const int idx = tid + e * NT;
      const int p = idx / XW;          // channel pair
      const int j = idx - p * XW;      // window position (consecutive threads: consecutive positions)
      const int ci = ci0 + 2 * p;
      const int t = tbase + j;
      float v0 = 0.f, v1 = 0.f;
      if (idx < npair && t >= 0 && t < a.L_in) {
        if (ci < ci_hi) v0 = xb[(long long)ci * a.xc + t];
        if (ci + 1 < ci_hi) v1 = xb[(long long)(ci + 1) * a.xc + t];
      }
      xr[e] = make_float2(v0, v1);
    }
#pragma unroll
    for (int e = 0; e < WPT; ++e) {
      const int idx = tid + e * NT;
      const int v = idx % WV;
      const int row = idx / WV;        // k * BM + co_local
      const int k = row / BM;
      const int co = co0 + (row - k * BM);
      const int ci = ci0 + 8 * v;
      uint4 w = make_uint4(0u, 0u, 0u, 0u);
      if (idx < nwv && co < a.C_out && ci < ci_hi)
        w = *reinterpret_cast<const uint4*>(G.w16 + ((long long)k * a.C_out + co) * a.w16_ld + ci);
      wreg[e] = w;
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int e = 0; e < XPT; ++e) {
      const int idx = tid + e * NT;
      if (idx < npair) {
        const int p = idx / XW;
        const int j = idx - p * XW;
        float v0 = xr[e].x, v1 = xr[e].y;
        if (a.in_act == ACT_LEAKY) {
          v0 = v0 >= 0.f ? v0 : v0 * a.in_slope;
          v1 = v1 >= 0.f ? v1 : v1 * a.in_slope;
        }
        *reinterpret_cast<uint32_t*>(xs + j * RS + 2 * p) = pack_bf16x2(v0, v1);
      }
    }
#pragma unroll
    for (int e = 0; e < WPT; ++e) {
      const int idx = tid + e * NT;
      if (idx < nwv) {
        const int v = idx % WV;
        const int row = idx / WV;
        *reinterpret_cast<uint4*>(ws + row * RS + 8 * v) = wreg[e];
      }
    }
  };

  if (K > 0 && ci_hi > ci_lo) {
    const int nchunk = (ci_hi - ci_lo + BKT - 1) / BKT;
    gload(ci_lo);
    for (int c = 0; c < nchunk; ++c) {
      lstore();
      __syncthreads();
      if (c + 1 < nchunk) gload(ci_lo + (c + 1) * BKT);
      for (int k = 0; k < K; ++k) {
        const uint16_t* wk_ = ws + (k * BM + wm * WM + l32) * RS + 8 * half;
        const uint16_t* xk = xs + (wn * WN + l32 + k * dil) * RS + 8 * half;
#pragma unroll
        for (int s16 = 0; s16 < BKT / 16; ++s16) {
          bf16x8 av[TM], bv[TN];
#pragma unroll
          for (int m = 0; m < TM; ++m) av[m] = as_bf16x8(*reinterpret_cast<const uint4*>(wk_ + m * 32 * RS + 16 * s16));
#pragma unroll
          for (int n = 0; n < TN; ++n) bv[n] = as_bf16x8(*reinterpret_cast<const uint4*>(xk + n * 32 * RS + 16 * s16));
#pragma unroll
          for (int m = 0; m < TM; ++m)
#pragma unroll
            for (int n = 0; n < TN; ++n)
              acc[m][n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[m], bv[n], acc[m][n], 0, 0, 0);
        }
      }
      __syncthreads();
    }
  }

  if (a.ksplit > 1) {
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

#pragma unroll
  for (int m = 0; m < TM; ++m) {
#pragma unroll
    for (int n = 0; n < TN; ++n) {
      const int i = i0 + wn * WN + n * 32 + l32;
      if (i >= G.n_out) continue;
      const long long t = (long long)i * G.out_step + G.out_off;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int co = co0 + wm * WM + m * 32 + (r & 3) + 4 * half + 8 * (r >> 2);
        if (co >= a.C_out) continue;
        float v = act_b(acc[m][n][r], a.out_act, a.out_slope);
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

constexpr size_t kLdsLimitB = 65536;

int max_n_out_b(const ConvLaunch& a) {
  int n = 0;
  for (int g = 0; g < a.n_groups; ++g) n = std::max(n, a.g[g].n_out);
  return n;
}

long long n_blocks_b(const ConvLaunch& a, int BM, int BN) {
  long long n = 0;
  for (int g = 0; g < a.n_groups; ++g) n += (long long)((a.g[g].n_out + BN - 1) / BN) * ((a.C_out + BM - 1) / BM);
  return n;
}

template <int BM, int BN, int WM, int WN, int BKT, int KMAX>
bool launch_b(const ConvLaunch& a, hipStream_t s) {
  using C = CfgB<BM, BN, WM, WN, BKT, KMAX>;
  size_t lds = 0;
  for (int g = 0; g < a.n_groups; ++g) {
    if (a.g[g].K > KMAX) return false;
    lds = std::max(lds, C::lds_bytes(a.g[g].K, a.g[g].dil));
  }
  if (lds > kLdsLimitB) return false;
  dim3 grid((max_n_out_b(a) + BN - 1) / BN, (a.C_out + BM - 1) / BM, a.n_groups * a.B * std::max(a.ksplit, 1));
  hipLaunchKernelGGL((conv1d_bf16_kernel<BM, BN, WM, WN, BKT, KMAX>), grid, dim3(C::NT), lds, s, a);
  check_launch("conv1d_bf16");
  if (a.ksplit > 1) launch_splitk_reduce(a, s);
  return true;
}

struct SplitB {
  int S = 1, csplit = 0;
};
// Split-K for a single-group launch whose tiles alone cannot fill the GPU
// (enc_p at P = 1000): whole 32-channel chunks, tiles x S near 640.  Like the
// fp32 plan it depends on the per-item tile count only, never on B.
SplitB split_b(const ConvLaunch& a) {
  SplitB p;
  if (a.n_groups != 1 || a.g[0].K < 1 || a.C_out % 64 != 0) return p;
  const int BM = a.C_out % 128 == 0 ? 128 : 64;
  const long long nb = n_blocks_b(a, BM, 128);
  if (nb >= 384) return p;
  const int BKT = 32;
  const int max_s = a.C_in / (2 * BKT);
  const int S = (int)std::min<long long>((640 + nb - 1) / nb, max_s);
  if (S < 2) return p;
  const int chunks = (a.C_in + BKT - 1) / BKT;
  const int per = (chunks + S - 1) / S;
  p.csplit = per * BKT;
  p.S = (a.C_in + p.csplit - 1) / p.csplit;
  return p;
}

}  // namespace

bool conv1d_bf16_supported(int K, int dil) {
  return K >= 0 && K <= kConvTapsMax && dil >= 1 && (K > 0 ? (K - 1) * dil : 0) <= kConvHaloMax;
}

size_t conv1d_bf16_split_floats(const ConvLaunch& a) {
  const SplitB p = split_b(a);
  return p.S > 1 ? (size_t)p.S * a.B * a.C_out * a.g[0].n_out : 0;
}

void launch_conv1d_bf16(const ConvLaunch& a, hipStream_t s) {
  RVC_CHECK(a.n_groups >= 1 && a.n_groups <= kMaxConvGroups, "conv1d_bf16: bad group count");
  RVC_CHECK(a.C_in >= 1 && a.C_out >= 1 && a.B >= 1 && a.w16_ld >= a.C_in && a.w16_ld % 8 == 0,
            "conv1d_bf16: invalid shape or weight row length");
  int kmax = 0;
  for (int g = 0; g < a.n_groups; ++g) {
    const ConvGroup& G = a.g[g];
    RVC_CHECK(G.w16 != nullptr, "conv1d_bf16: group without bf16 weights");
    RVC_CHECK(G.in_step <= 1, "conv1d_bf16: input stride 1 only");
    RVC_CHECK(G.n_out >= 0 && conv1d_bf16_supported(G.K, G.dil), "conv1d_bf16: taps / dilation outside the kernel");
    RVC_CHECK((reinterpret_cast<uintptr_t>(G.w16) & 15) == 0, "conv1d_bf16: weights must be 16-byte aligned");
    kmax = std::max(kmax, G.K);
  }
  if (max_n_out_b(a) == 0) return;
  if (a.part && a.part_floats > 0) {
    const SplitB p = split_b(a);
    if (p.S > 1 && (size_t)p.S * a.B * a.C_out * a.g[0].n_out <= a.part_floats) {
      ConvLaunch sa = a;
      sa.ksplit = p.S;
      sa.csplit = p.csplit;
      // (the split tiles take up to 3 taps; longer convs run unsplit below)
      const bool ok = a.C_out % 128 == 0 ? launch_b<128, 128, 64, 64, 32, 3>(sa, s) : launch_b<64, 128, 32, 64, 32, 3>(sa, s);
      if (ok) return;
    }
  }
  const long long want = 384;
  bool ok = false;
  if (kmax <= 1) {
    if (a.C_out % 128 == 0 && n_blocks_b(a, 128, 128) >= want) ok = launch_b<128, 128, 64, 64, 64, 1>(a, s);
    if (!ok && a.C_out % 64 == 0 && n_blocks_b(a, 64, 128) >= want) ok = launch_b<64, 128, 32, 64, 64, 1>(a, s);
  } else if (kmax <= 3) {
    if (a.C_out % 128 == 0 && n_blocks_b(a, 128, 128) >= want) ok = launch_b<128, 128, 64, 64, 32, 3>(a, s);
    if (!ok && a.C_out % 64 == 0 && n_blocks_b(a, 64, 128) >= want) ok = launch_b<64, 128, 32, 64, 32, 3>(a, s);
  }
  if (!ok && a.C_out % 64 == 0 && n_blocks_b(a, 64, 128) >= want) ok = launch_b<64, 128, 32, 64, 16, 11>(a, s);
  if (!ok && a.C_out <= 32 && n_blocks_b(a, 32, 256) >= want) ok = launch_b<32, 256, 32, 64, 16, 11>(a, s);
  if (!ok) ok = launch_b<32, 64, 32, 32, 16, 11>(a, s);
  RVC_CHECK(ok, "conv1d_bf16: no tile configuration fits the LDS budget");
}

}  // namespace rvc
