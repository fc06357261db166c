// LayerNorm and softmax.
//
// LayerNorm is the two-pass biased-variance form of the reference numpy
// path, (x - mean) / sqrt(var + eps) * gamma + beta (runtime/backend.py:
// 286-295) -- not the single-pass E[x^2]-E[x]^2 of the reference's GLSL
// (engine/shaders/layernorm.comp:68-70).  Sums accumulate in double.
// Softmax is exp(x - max) / sum (runtime/backend.py:298-306).
#include "internal.h"

#pragma clang fp contract(off)

namespace rvc {
namespace {

__device__ double block_sum_d(double v, double* sh) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) sh[w] = v;
  __syncthreads();
  double t = 0.0;
  const int nw = blockDim.x >> 6;
  for (int i = 0; i < nw; ++i) t += sh[i];
  return t;
}

__device__ float block_max_f(float v, float* sh) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) sh[w] = v;
  __syncthreads();
  float t = sh[0];
  const int nw = blockDim.x >> 6;
  for (int i = 1; i < nw; ++i) t = fmaxf(t, sh[i]);
  return t;
}

// One workgroup per row of a row-major [rows][cols] tensor.
__global__ __launch_bounds__(256) void layernorm_rows_kernel(const float* x, const float* g, const float* b,
                                                             float* out, int cols, float eps) {
  __shared__ double sh[8];
  const long long row = blockIdx.x;
  const float* xr = x + row * cols;
  float* orow = out + row * cols;
  double s = 0.0;
  for (int c = threadIdx.x; c < cols; c += blockDim.x) s += xr[c];
  const float mean = (float)(block_sum_d(s, sh) / cols);
  double v = 0.0;
  for (int c = threadIdx.x; c < cols; c += blockDim.x) {
    const float d = xr[c] - mean;
    v += (double)d * d;
  }
  const float var = (float)(block_sum_d(v, sh) / cols);
  const float den = sqrtf(var + eps);
  for (int c = threadIdx.x; c < cols; c += blockDim.x) orow[c] = (xr[c] - mean) / den * g[c] + b[c];
}

// Channel-major LayerNorm with one wavefront per column (b, t): the C values
// sit in registers (NR per lane, C <= 64 * NR), the two reductions are wave
// shuffles, so each column costs one read and one write pass and the grid
// has B * L / 4 workgroups (enough to spread a 499-frame layer over the CUs).
// Same formulas as layernorm_cols_kernel.
template <int NR>
__global__ __launch_bounds__(256) void layernorm_cols_wave_kernel(const float* x, const float* g, const float* b,
                                                                  float* out, int C, int L, float eps) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= L) return;  // whole wave; no workgroup barrier below
  const long long base = (long long)blockIdx.y * C * L + t;
  float v[NR];
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int c = lane + 64 * i;
    v[i] = c < C ? x[base + (long long)c * L] : 0.f;
    s += v[i];
  }
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  const float mean = (float)(s / C);
  double q = 0.0;
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int c = lane + 64 * i;
    if (c < C) {
      const float d = v[i] - mean;
      q += (double)d * d;
    }
  }
  for (int o = 32; o > 0; o >>= 1) q += __shfl_xor(q, o);
  const float den = sqrtf((float)(q / C) + eps);
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int c = lane + 64 * i;
    if (c < C) out[base + (long long)c * L] = (v[i] - mean) / den * g[c] + b[c];
  }
}

// GroupNorm with one channel per group on [B][C][L] (the normalisation runs
// over L for each (b, c)), two-pass in float64 like the row LayerNorm, then
// the per-channel affine and an activation:
//   out = act((x - mean) / sqrt(var + eps) * g[c] + b[c])
// (runtime/nn.py:415-436 with num_groups == C, then gelu_erf for HuBERT's
// first feature-extractor layer, runtime/models/hubert.py:686-692).
__global__ __launch_bounds__(256) void groupnorm_rows_act_kernel(const float* x, const float* g, const float* b,
                                                                 float* out, int C, long long L, float eps, int act) {
  __shared__ double sh[256 / 64];
  const long long row = blockIdx.x;
  const int c = (int)(row % C);
  const float* xr = x + row * L;
  float* orow = out + row * L;
  double s = 0.0;
  for (long long i = threadIdx.x; i < L; i += blockDim.x) s += xr[i];
  const float mean = (float)(block_sum_d(s, sh) / (double)L);
  double v = 0.0;
  for (long long i = threadIdx.x; i < L; i += blockDim.x) {
    const float d = xr[i] - mean;
    v += (double)d * d;
  }
  const float var = (float)(block_sum_d(v, sh) / (double)L);
  const float den = sqrtf(var + eps);
  const float gc = g[c], bc = b[c];
  for (long long i = threadIdx.x; i < L; i += blockDim.x) {
    float y = (xr[i] - mean) / den * gc + bc;
    if (act == ACT_GELU) y = gelu_as(y);
    orow[i] = y;
  }
}

// The same GroupNorm for rows of at most NT * NPT values, held in registers
// (thread t keeps elements t + NT j): one read and one write pass instead of
// three reads, with the same operations per element.  HuBERT's first
// GroupNorm (512 rows of 31 999) runs 1024 threads x 32 values per row: 16
// waves per CU keep more loads in flight than 256 x 128 (4.1 against 3.1
// TB/s, 48 against 64 us).
template <int NPT, int NT>
__global__ __launch_bounds__(NT) void groupnorm_rows_act_reg_kernel(const float* x, const float* g, const float* b,
                                                                    float* out, int C, int L, float eps, int act) {
  __shared__ double sh[NT / 64];
  const long long row = blockIdx.x;
  const int c = (int)(row % C);
  const int tid = threadIdx.x;
  // element tid + NT j through a resource over [NT j, L) of the row, so
  // the per-element offset is the one register 4 * tid and the range check
  // zeroes (and drops) everything past L
  auto part = [&](const float* base, int j) {
    return uniform_rsrc(base + row * L + NT * j, 4u * (unsigned)max(L - NT * j, 0));
  };
  float v[NPT];
#pragma unroll
  for (int j = 0; j < NPT; ++j)
    v[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(part(x, j), 4u * (unsigned)tid, 0, 0));
  double s = 0.0;
#pragma unroll
  for (int j = 0; j < NPT; ++j)
    if (tid + NT * j < L) s += v[j];
  const float mean = (float)(block_sum_d(s, sh) / (double)L);
  double q = 0.0;
#pragma unroll
  for (int j = 0; j < NPT; ++j)
    if (tid + NT * j < L) {
      const float d = v[j] - mean;
      q += (double)d * d;
    }
  const float var = (float)(block_sum_d(q, sh) / (double)L);
  const float den = sqrtf(var + eps);
  const float gc = g[c], bc = b[c];
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    float y = (v[j] - mean) / den * gc + bc;
    if (act == ACT_GELU) y = gelu_as(y);
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, y), part(out, j), 4u * (unsigned)tid, 0, 0);
  }
}

// GroupNorm of the op-level ABI: x is [G][Cpg*S] (G groups, Cpg channels of
// S elements each); every row is standardised over its Cpg*S values and
// element i of row g gets the affine of channel g*Cpg + i/S
// (engine/shaders/gn.comp:1-8).  Statistics two-pass in double.
__global__ __launch_bounds__(256) void groupnorm_groups_kernel(const float* x, const float* g, const float* b,
                                                               float* out, int Cpg, long long S, float eps) {
  __shared__ double sh[256 / 64];
  const long long row = blockIdx.x;
  const long long n = (long long)Cpg * S;
  const float* xr = x + row * n;
  float* orow = out + row * n;
  double s = 0.0;
  for (long long i = threadIdx.x; i < n; i += blockDim.x) s += xr[i];
  const float mean = (float)(block_sum_d(s, sh) / (double)n);
  double v = 0.0;
  for (long long i = threadIdx.x; i < n; i += blockDim.x) {
    const float d = xr[i] - mean;
    v += (double)d * d;
  }
  const float var = (float)(block_sum_d(v, sh) / (double)n);
  const float den = sqrtf(var + eps);
  const long long c0 = row * Cpg;
  for (long long i = threadIdx.x; i < n; i += blockDim.x) {
    const long long c = c0 + i / S;
    orow[i] = (xr[i] - mean) / den * g[c] + b[c];
  }
}

// RMSNorm over the last dim: out = x * (1 / sqrt(mean(x^2) + eps)) * gamma
// (engine/shaders/rmsnorm.comp:1-6); the sum of squares accumulates in double.
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const float* x, const float* g, float* out, int cols,
                                                           float eps) {
  __shared__ double sh[256 / 64];
  const long long row = blockIdx.x;
  const float* xr = x + row * cols;
  float* orow = out + row * cols;
  double q = 0.0;
  for (int i = threadIdx.x; i < cols; i += blockDim.x) q += (double)xr[i] * xr[i];
  const float inv = 1.0f / sqrtf((float)(block_sum_d(q, sh) / (double)cols) + eps);
  for (int i = threadIdx.x; i < cols; i += blockDim.x) orow[i] = xr[i] * inv * g[i];
}

// Channel-major [B][C][L]: normalise over C for each (b, t).  A workgroup
// owns LN_COLS consecutive columns; its LN_GRP thread groups split the
// channels (coalesced reads along t) and combine partial sums in LDS.
constexpr int LN_COLS = 32;
constexpr int LN_GRP = 8;

__global__ __launch_bounds__(LN_COLS * LN_GRP) void layernorm_cols_kernel(const float* x, const float* g,
                                                                          const float* b, float* out, int C,
                                                                          int L, float eps) {
  __shared__ double part[LN_GRP][LN_COLS];
  __shared__ float stat[2][LN_COLS];
  const int tx = threadIdx.x % LN_COLS;
  const int ty = threadIdx.x / LN_COLS;
  const int t = blockIdx.x * LN_COLS + tx;
  const long long base = (long long)blockIdx.y * C * L;
  const bool ok = t < L;
  const float* xc = x + base + t;
  double s = 0.0;
  if (ok)
    for (int c = ty; c < C; c += LN_GRP) s += xc[(long long)c * L];
  part[ty][tx] = s;
  __syncthreads();
  if (ty == 0) {
    double tot = 0.0;
    for (int i = 0; i < LN_GRP; ++i) tot += part[i][tx];
    stat[0][tx] = (float)(tot / C);
  }
  __syncthreads();
  const float mean = stat[0][tx];
  double v = 0.0;
  if (ok)
    for (int c = ty; c < C; c += LN_GRP) {
      const float d = xc[(long long)c * L] - mean;
      v += (double)d * d;
    }
  part[ty][tx] = v;
  __syncthreads();
  if (ty == 0) {
    double tot = 0.0;
    for (int i = 0; i < LN_GRP; ++i) tot += part[i][tx];
    stat[1][tx] = sqrtf((float)(tot / C) + eps);
  }
  __syncthreads();
  const float den = stat[1][tx];
  if (ok) {
    float* oc = out + base + t;
    for (int c = ty; c < C; c += LN_GRP) oc[(long long)c * L] = (xc[(long long)c * L] - mean) / den * g[c] + b[c];
  }
}

__global__ __launch_bounds__(256) void softmax_rows_kernel(const float* x, float* out, int cols) {
  __shared__ float shf[8];
  __shared__ double shd[8];
  const long long row = blockIdx.x;
  const float* xr = x + row * cols;
  float* orow = out + row * cols;
  float m = -INFINITY;
  for (int c = threadIdx.x; c < cols; c += blockDim.x) m = fmaxf(m, xr[c]);
  m = block_max_f(m, shf);
  double s = 0.0;
  for (int c = threadIdx.x; c < cols; c += blockDim.x) {
    const float e = expf(xr[c] - m);
    orow[c] = e;
    s += e;
  }
  const float sum = (float)block_sum_d(s, shd);
  for (int c = threadIdx.x; c < cols; c += blockDim.x) orow[c] = orow[c] / sum;
}

}  // namespace

void launch_layernorm_rows(const float* x, const float* g, const float* b, float* out, long long rows,
                           int cols, float eps, hipStream_t s) {
  if (rows <= 0 || cols <= 0) return;
  RVC_CHECK(rows <= 0x7fffffffLL, "layernorm: too many rows");
  hipLaunchKernelGGL(layernorm_rows_kernel, dim3((unsigned)rows), dim3(256), 0, s, x, g, b, out, cols, eps);
  check_launch("layernorm_rows");
}

void launch_layernorm_cols(const float* x, const float* g, const float* b, float* out, int B, int C, int L,
                           float eps, hipStream_t s) {
  if ((long long)B * L <= 0 || C <= 0) return;
  if (C <= 1024) {
    dim3 grid((L + 3) / 4, B);
    if (C <= 256)
      hipLaunchKernelGGL(layernorm_cols_wave_kernel<4>, grid, dim3(256), 0, s, x, g, b, out, C, L, eps);
    else if (C <= 512)
      hipLaunchKernelGGL(layernorm_cols_wave_kernel<8>, grid, dim3(256), 0, s, x, g, b, out, C, L, eps);
    else
      hipLaunchKernelGGL(layernorm_cols_wave_kernel<16>, grid, dim3(256), 0, s, x, g, b, out, C, L, eps);
  } else {
    dim3 grid((L + LN_COLS - 1) / LN_COLS, B);
    hipLaunchKernelGGL(layernorm_cols_kernel, grid, dim3(LN_COLS * LN_GRP), 0, s, x, g, b, out, C, L, eps);
  }
  check_launch("layernorm_cols");
}

void launch_groupnorm_rows_act(const float* x, const float* g, const float* b, float* out, int B, int C, long long L,
                               float eps, int act, hipStream_t s) {
  if (B <= 0 || C <= 0 || L <= 0) return;
  if (L <= 1024 * 32) {
    hipLaunchKernelGGL((groupnorm_rows_act_reg_kernel<32, 1024>), dim3((unsigned)((long long)B * C)), dim3(1024), 0, s,
                       x, g, b, out, C, (int)L, eps, act);
    check_launch("groupnorm_rows_act");
    return;
  }
  hipLaunchKernelGGL(groupnorm_rows_act_kernel, dim3((unsigned)((long long)B * C)), dim3(256), 0, s, x, g, b, out, C,
                     L, eps, act);
  check_launch("groupnorm_rows_act");
}

void launch_groupnorm_groups(const float* x, const float* g, const float* b, float* out, long long G, int Cpg,
                             long long S, float eps, hipStream_t s) {
  if (G <= 0 || Cpg <= 0 || S <= 0) return;
  RVC_CHECK(G <= 0x7fffffffLL, "group_norm: too many groups");
  hipLaunchKernelGGL(groupnorm_groups_kernel, dim3((unsigned)G), dim3(256), 0, s, x, g, b, out, Cpg, S, eps);
  check_launch("groupnorm_groups");
}

void launch_rmsnorm_rows(const float* x, const float* g, float* out, long long rows, int cols, float eps,
                         hipStream_t s) {
  if (rows <= 0 || cols <= 0) return;
  RVC_CHECK(rows <= 0x7fffffffLL, "rmsnorm: too many rows");
  hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3((unsigned)rows), dim3(256), 0, s, x, g, out, cols, eps);
  check_launch("rmsnorm_rows");
}

void launch_softmax_rows(const float* x, float* out, long long rows, int cols, hipStream_t s) {
  if (rows <= 0 || cols <= 0) return;
  RVC_CHECK(rows <= 0x7fffffffLL, "softmax: too many rows");
  hipLaunchKernelGGL(softmax_rows_kernel, dim3((unsigned)rows), dim3(256), 0, s, x, out, cols);
  check_launch("softmax_rows");
}

}  // namespace rvc
