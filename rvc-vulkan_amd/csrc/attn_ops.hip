// Op-level attention kernels of the record/commit ABI (batch op codes 12, 13,
// 16, 17; engine/src/ffi.zig:899-912).  q, k, v are [T][C] with head h in
// columns [h*D, (h+1)*D) ("head-interleaved"), scores / weights are
// [H][T][T], and `used` [2T-1][D] is the relative-position table indexed by
// m = s - t + T - 1 (the banded forms):
//
//   scores[h,t,s] = sum_d q[t,hD+d] * (k[s,hD+d] + used[m,d])        (16; 12 without used)
//   ctx[t,hD+d]   = sum_s W[h,t,s]  * (v[s,hD+d] + used[m,d])        (17; 13 without used)
//
// The synthesis session does not use these (its fused flash-style kernel in
// attention.hip never materialises [H][T][T]); they exist so the reference's
// vulkan_ops-style callers can drive the same ops through this library.
//
// Both are LDS-tiled fp32 SIMT kernels: a 256-thread workgroup owns a 64x64
// output tile, each thread a 4x4 block (rows ty+16i, columns tx+16j), and the
// reduction axis advances in chunks of 16 staged in LDS together with the
// slice of `used` the tile's diagonals touch (127 rows for scores, 79 rows
// for the context).  Each output sums its reduction axis in order, one term
// at a time, like the reference shaders (engine/shaders/banded_attn_qk.comp,
// banded_attn_sv.comp).
#include "internal.h"

#pragma clang fp contract(off)

namespace rvc {
namespace {

constexpr int TILE = 64;
constexpr int CH = 16;

template <bool BANDED>
__global__ __launch_bounds__(256) void attn_scores_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                          const float* __restrict__ used, float* __restrict__ out,
                                                          int T, int D, int C) {
  __shared__ float sQ[CH][TILE + 1];
  __shared__ float sK[CH][TILE + 1];
  __shared__ float sU[BANDED ? CH : 1][2 * TILE];
  const int tid = threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;
  const int s0 = blockIdx.x * TILE, t0 = blockIdx.y * TILE, h = blockIdx.z;
  const long long hd = (long long)h * D;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;

  for (int d0 = 0; d0 < D; d0 += CH) {
    // q / k tiles: consecutive threads read consecutive d of one row
#pragma unroll
    for (int r = 0; r < (CH * TILE) / 256; ++r) {
      const int e = tid + 256 * r;
      const int dd = e & (CH - 1), row = e / CH;
      const int d = d0 + dd;
      const int t = t0 + row, s = s0 + row;
      sQ[dd][row] = (t < T && d < D) ? q[(long long)t * C + hd + d] : 0.f;
      sK[dd][row] = (s < T && d < D) ? k[(long long)s * C + hd + d] : 0.f;
    }
    if (BANDED) {
      // sU[dd][j] = used[(s0 - t0) + j - (TILE-1) + T - 1][d0 + dd], j in [0, 2*TILE-1)
      for (int e = tid; e < CH * (2 * TILE - 1); e += 256) {
        const int dd = e & (CH - 1), j = e / CH;
        const int d = d0 + dd;
        const long long m = (long long)(s0 - t0) + j - (TILE - 1) + T - 1;
        sU[dd][j] = (m >= 0 && m <= 2LL * T - 2 && d < D) ? used[m * D + d] : 0.f;
      }
    }
    __syncthreads();
#pragma unroll 4
    for (int dd = 0; dd < CH; ++dd) {
      float qv[4], kv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) qv[i] = sQ[dd][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) kv[j] = sK[dd][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float kk = kv[j];
          if (BANDED) kk = kk + sU[dd][(tx + 16 * j) - (ty + 16 * i) + TILE - 1];
          acc[i][j] = acc[i][j] + qv[i] * kk;
        }
    }
    __syncthreads();
  }
  float* oh = out + (long long)h * T * T;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = t0 + ty + 16 * i;
    if (t >= T) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int s = s0 + tx + 16 * j;
      if (s < T) oh[(long long)t * T + s] = acc[i][j];
    }
  }
}

template <bool BANDED>
__global__ __launch_bounds__(256) void attn_context_kernel(const float* __restrict__ w, const float* __restrict__ v,
                                                           const float* __restrict__ used, float* __restrict__ out,
                                                           int T, int D, int C) {
  constexpr int UR = TILE + CH - 1;  // diagonals one s chunk meets: s - t in [sc - t0 - 63, sc - t0 + 15]
  __shared__ float sW[CH][TILE + 1];
  __shared__ float sV[CH][TILE];
  __shared__ float sU[BANDED ? UR : 1][TILE];
  const int tid = threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;
  const int d0 = blockIdx.x * TILE, t0 = blockIdx.y * TILE, h = blockIdx.z;
  const long long hd = (long long)h * D;
  const float* wh = w + (long long)h * T * T;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;

  for (int sc = 0; sc < T; sc += CH) {
#pragma unroll
    for (int r = 0; r < (CH * TILE) / 256; ++r) {
      const int e = tid + 256 * r;
      {  // weights: consecutive threads along s of one row t
        const int sl = e & (CH - 1), tl = e / CH;
        const int t = t0 + tl, s = sc + sl;
        sW[sl][tl] = (t < T && s < T) ? wh[(long long)t * T + s] : 0.f;
      }
      {  // values: consecutive threads along d of one row s
        const int dl = e & (TILE - 1), sl = e / TILE;
        const int s = sc + sl, d = d0 + dl;
        sV[sl][dl] = (s < T && d < D) ? v[(long long)s * C + hd + d] : 0.f;
      }
    }
    if (BANDED) {
      // sU[j][dl] = used[(sc - t0) + j - (TILE-1) + T - 1][d0 + dl]
      for (int e = tid; e < UR * TILE; e += 256) {
        const int dl = e & (TILE - 1), j = e / TILE;
        const int d = d0 + dl;
        const long long m = (long long)(sc - t0) + j - (TILE - 1) + T - 1;
        sU[j][dl] = (m >= 0 && m <= 2LL * T - 2 && d < D) ? used[m * D + d] : 0.f;
      }
    }
    __syncthreads();
#pragma unroll 4
    for (int sl = 0; sl < CH; ++sl) {
      float wv[4], vv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) wv[i] = sW[sl][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) vv[j] = sV[sl][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float vx = vv[j];
          if (BANDED) vx = vx + sU[sl - (ty + 16 * i) + TILE - 1][tx + 16 * j];
          acc[i][j] = acc[i][j] + wv[i] * vx;
        }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = t0 + ty + 16 * i;
    if (t >= T) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = d0 + tx + 16 * j;
      if (d < D) out[(long long)t * C + hd + d] = acc[i][j];
    }
  }
}

void check_dims(int H, int T, int D, int C, const char* what) {
  RVC_CHECK(H >= 1 && T >= 1 && D >= 1 && (long long)H * D <= C, std::string(what) + ": need H, T, D >= 1 and H*D <= C");
  RVC_CHECK((T + TILE - 1) / TILE <= 65535 && H <= 65535, std::string(what) + ": T or H exceeds the launch grid");
}

}  // namespace

void launch_attn_scores(const float* q, const float* k, const float* used, float* out, int H, int T, int D, int C,
                        hipStream_t s) {
  check_dims(H, T, D, C, "attn_qk");
  const dim3 grid((T + TILE - 1) / TILE, (T + TILE - 1) / TILE, H);
  if (used)
    hipLaunchKernelGGL(attn_scores_kernel<true>, grid, dim3(256), 0, s, q, k, used, out, T, D, C);
  else
    hipLaunchKernelGGL(attn_scores_kernel<false>, grid, dim3(256), 0, s, q, k, used, out, T, D, C);
  check_launch("attn_scores");
}

void launch_attn_context(const float* w, const float* v, const float* used, float* out, int H, int T, int D, int C,
                         hipStream_t s) {
  check_dims(H, T, D, C, "attn_sv");
  const dim3 grid((D + TILE - 1) / TILE, (T + TILE - 1) / TILE, H);
  if (used)
    hipLaunchKernelGGL(attn_context_kernel<true>, grid, dim3(256), 0, s, w, v, used, out, T, D, C);
  else
    hipLaunchKernelGGL(attn_context_kernel<false>, grid, dim3(256), 0, s, w, v, used, out, T, D, C);
  check_launch("attn_context");
}

}  // namespace rvc
