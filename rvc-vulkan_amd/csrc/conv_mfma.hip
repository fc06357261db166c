// Implicit-GEMM conv1d on CDNA4 fp32 matrix cores (v_mfma_f32_32x32x2_f32).
//
// out[b][co][i] = sum_{ci,k} W[k][ci][co] * act(x[b][ci][i + in_off + k*dil])
// viewed as a GEMM with M = C_out, N = output positions and a reduction over
// (ci, k).  One workgroup owns a BM x BN output tile.  For each chunk of BK
// input channels it stages, in LDS,
//   * the input window x[ci0:ci0+BK][i0+in_off : i0+in_off+BN+(K-1)*dil]
//     once -- every tap re-reads the same window at a shift of k*dil, so
//     the halo is loaded once per chunk instead of K times, and
//   * the packed weights W[0:K][ci0:ci0+BK][co0:co0+BM].
// Each wave computes a WM x WN sub-tile with (WM/32)*(WN/32) 32x32
// accumulators.  Per MFMA step (two input channels) lane l supplies
//   A = W[k][ci0+2q+l/32][co_tile + l%32]      (row = co, k-index = ci)
//   B = xs[2q+l/32][col_tile + l%32 + k*dil]    (k-index = ci, col = i)
// and the 16 accumulator registers r of lane l hold
//   row = (r%4) + 4*(l/32) + 8*(r/4), col = l%32.
// The fused epilogue adds bias (and an optional second per-channel term),
// an optional residual, applies leaky-ReLU/tanh and combines into the output
// (store, accumulate, or accumulate-then-divide for the ResBlock average).
// Output position i is written at i*out_step + out_off, which lets one phase
// of a polyphase ConvTranspose1d use the same kernel.
#include "internal.h"

namespace rvc {

typedef float floatx16 __attribute__((ext_vector_type(16)));

namespace {

__device__ __forceinline__ float apply_act(float v, int act, float slope) {
  if (act == ACT_LEAKY) return v >= 0.f ? v : v * slope;
  if (act == ACT_TANH) return tanhf(v);
  if (act == ACT_RELU) return fmaxf(v, 0.f);
  return v;
}

template <int BM, int BN, int WM, int WN, int BK>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void conv1d_mfma_kernel(ConvArgs a) {
  constexpr int NWM = BM / WM;
  constexpr int NWN = BN / WN;
  constexpr int NWAVES = NWM * NWN;
  constexpr int NT = NWAVES * 64;
  constexpr int TM = WM / 32;
  constexpr int TN = WN / 32;
  static_assert(BK % 2 == 0, "BK must be even");

  extern __shared__ float smem[];
  const int K = a.K;
  const int dil = a.dil;
  const int XW = BN + (K > 0 ? (K - 1) * dil : 0);
  float* xs = smem;            // [BK][XW]
  float* ws = smem + BK * XW;  // [K][BK][BM]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % NWM;
  const int wn = wave / NWM;
  const int b = blockIdx.z;
  const int i0 = blockIdx.x * BN;
  const int co0 = blockIdx.y * BM;
  const float* xb = a.x + (long long)b * a.xb;
  const int half = lane >> 5;
  const int l32 = lane & 31;

  floatx16 acc[TM][TN];
#pragma unroll
  for (int m = 0; m < TM; ++m)
#pragma unroll
    for (int n = 0; n < TN; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[m][n][r] = 0.f;

  for (int ci0 = 0; ci0 < a.C_in && K > 0; ci0 += BK) {
    // ---- stage the input window (prologue activation applied here) ----
    const int tbase = i0 + a.in_off;
    for (int r = 0; r < BK; ++r) {
      const int ci = ci0 + r;
      const bool cin = ci < a.C_in;
      const float* xr = xb + (long long)ci * a.xc;
      for (int j = tid; j < XW; j += NT) {
        const int t = tbase + j;
        float v = 0.f;
        if (cin && t >= 0 && t < a.L_in) {
          v = xr[t];
          if (a.in_act == ACT_LEAKY) v = v >= 0.f ? v : v * a.in_slope;
        }
        xs[r * XW + j] = v;
      }
    }
    // ---- stage the packed weights ----
    for (int row = wave; row < K * BK; row += NWAVES) {
      const int k = row / BK;
      const int r = row - k * BK;
      const int ci = ci0 + r;
      const float* wr = a.w + ((long long)k * a.C_in + ci) * a.C_out + co0;
      for (int c = lane; c < BM; c += 64) {
        float v = 0.f;
        if (ci < a.C_in && co0 + c < a.C_out) v = wr[c];
        ws[row * BM + c] = v;
      }
    }
    __syncthreads();

    for (int k = 0; k < K; ++k) {
      const float* wk = ws + k * BK * BM + wm * WM + l32;
      const float* xk = xs + wn * WN + l32 + k * dil;
#pragma unroll
      for (int q = 0; q < BK / 2; ++q) {
        const int r = 2 * q + half;
        float av[TM], bv[TN];
#pragma unroll
        for (int m = 0; m < TM; ++m) av[m] = wk[r * BM + m * 32];
#pragma unroll
        for (int n = 0; n < TN; ++n) bv[n] = xk[r * XW + n * 32];
#pragma unroll
        for (int m = 0; m < TM; ++m)
#pragma unroll
          for (int n = 0; n < TN; ++n)
            acc[m][n] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[m], bv[n], acc[m][n], 0, 0, 0);
      }
    }
    __syncthreads();
  }

  // ---- fused epilogue ----
  const float* bias2 = a.bias2 ? a.bias2 + (long long)b * a.bias2b : nullptr;
  float* ob = a.out + (long long)b * a.ob;
  const float* rb = a.res ? a.res + (long long)b * a.rb : nullptr;
#pragma unroll
  for (int m = 0; m < TM; ++m) {
#pragma unroll
    for (int n = 0; n < TN; ++n) {
      const int i = i0 + wn * WN + n * 32 + l32;
      if (i >= a.n_out) continue;
      const long long t = (long long)i * a.out_step + a.out_off;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = (r & 3) + 4 * half + 8 * (r >> 2);
        const int co = co0 + wm * WM + m * 32 + row;
        if (co >= a.C_out) continue;
        float v = acc[m][n][r];
        if (a.bias) v = v + a.bias[co];
        if (bias2) v = v + bias2[co];
        if (rb) v = v + rb[co * a.rc + t];
        v = apply_act(v, a.out_act, a.out_slope);
        float* o = ob + co * a.oc + t;
        if (a.combine == COMB_ADD) {
          v = *o + v;
        } else if (a.combine == COMB_ADD_DIV) {
          v = (*o + v) / a.div;
        }
        *o = v;
      }
    }
  }
}

template <int BM, int BN, int WM, int WN, int BK>
void launch_cfg(const ConvArgs& a, hipStream_t s) {
  constexpr int NT = (BM / WM) * (BN / WN) * 64;
  const int XW = BN + (a.K > 0 ? (a.K - 1) * a.dil : 0);
  const size_t lds = sizeof(float) * ((size_t)BK * XW + (size_t)a.K * BK * BM);
  dim3 grid((a.n_out + BN - 1) / BN, (a.C_out + BM - 1) / BM, a.B);
  hipLaunchKernelGGL((conv1d_mfma_kernel<BM, BN, WM, WN, BK>), grid, dim3(NT), lds, s, a);
  check_launch("conv1d_mfma");
}

size_t lds_bytes(int BM, int BN, int BK, int K, int dil) {
  const int XW = BN + (K > 0 ? (K - 1) * dil : 0);
  return sizeof(float) * ((size_t)BK * XW + (size_t)K * BK * BM);
}

constexpr size_t kLdsLimit = 65536;

template <int BM, int BN, int WM, int WN>
bool try_launch(const ConvArgs& a, hipStream_t s) {
  if (lds_bytes(BM, BN, 16, a.K, a.dil) <= kLdsLimit) {
    launch_cfg<BM, BN, WM, WN, 16>(a, s);
    return true;
  }
  if (lds_bytes(BM, BN, 8, a.K, a.dil) <= kLdsLimit) {
    launch_cfg<BM, BN, WM, WN, 8>(a, s);
    return true;
  }
  if (lds_bytes(BM, BN, 2, a.K, a.dil) <= kLdsLimit) {
    launch_cfg<BM, BN, WM, WN, 2>(a, s);
    return true;
  }
  return false;
}

long long n_blocks(const ConvArgs& a, int BM, int BN) {
  return (long long)((a.n_out + BN - 1) / BN) * ((a.C_out + BM - 1) / BM) * a.B;
}

}  // namespace

void launch_conv1d_mfma(const ConvArgs& a, hipStream_t s) {
  RVC_CHECK(a.C_in >= 1 && a.C_out >= 1 && a.n_out >= 0 && a.K >= 0 && a.dil >= 1 && a.B >= 1,
            "conv1d_mfma: invalid shape");
  if (a.n_out == 0) return;
  // Tile choice: the widest co tile that divides C_out, shrunk while the grid
  // would leave CUs idle (256 CUs; aim for >= 2 workgroups per CU).
  const long long want = 512;
  bool ok = false;
  if (a.C_out % 128 == 0 && n_blocks(a, 128, 128) >= want) {
    ok = try_launch<128, 128, 64, 64>(a, s);
  } else if (a.C_out % 64 == 0 && n_blocks(a, 64, 128) >= want) {
    ok = try_launch<64, 128, 32, 64>(a, s);
  } else if (a.C_out % 64 == 0) {
    ok = try_launch<64, 64, 32, 32>(a, s);
  } else if (a.C_out <= 32 && n_blocks(a, 32, 256) >= want) {
    ok = try_launch<32, 256, 32, 64>(a, s);
  } else {
    ok = try_launch<32, 128, 32, 32>(a, s);
  }
  RVC_CHECK(ok, "conv1d_mfma: kernel window does not fit in LDS (K*dil too large)");
}

}  // namespace rvc
