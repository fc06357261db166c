// HuBERT's positional convolution (runtime/models/hubert.py:838-858): a
// grouped Conv1d with few channels per group and a long kernel (base model:
// 16 groups of 48 channels, 128 taps, padding 64, the last output column
// dropped), on fp32 matrix cores (v_mfma_f32_16x16x4_f32):
//
//   out[b][g*CPG + co][t] = bias[g*CPG + co]
//       + sum_{k < K} sum_{ci < CPG} W[g][k][ci][co] * x[b][g*CPG + ci][t + k - pad]
//
// A workgroup owns one group and kTT = 32 output columns, all CPG output
// channels.  The input window of those columns (CPG rows x kTT + K - 1
// columns, zero outside [0, L)) is staged once and every tap reads it at a
// shift; the weights stream through LDS one tap per part per step, double
// buffered, by direct-to-LDS loads.  The taps are cut into kNQ parts of K /
// kNQ; waves 2q and 2q + 1 take part q, each for one 16-column half of the
// tile and all CPG / 16 row tiles; the parts' sums are added through LDS in
// part order (((p0 + p1) + p2) + p3), then the bias.  One launch replaces the
// tap-block launches of the general convolution (11 taps each, every one
// re-reading and re-writing the output).
#include "internal.h"

namespace rvc {

typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kTT = 32;        // output columns per workgroup
constexpr int kNQ = 4;         // tap parts (two waves each: the two 16-column halves)
constexpr int kKB = 1;         // taps per part per staging step
constexpr int kNT = kNQ * 128;

template <int CPG>
__global__ __launch_bounds__(kNT) void posconv_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                      const float* __restrict__ bias, float* __restrict__ out,
                                                      int H, int L, int K, int pad) {
  constexpr int TM = CPG / 16;            // 16-row tiles
  constexpr int TAPW = CPG * CPG;         // floats of one tap's [ci][co] block
  constexpr int STEPW = kNQ * kKB * TAPW;  // one staging step: kNQ parts x kKB taps
  static_assert(CPG % 16 == 0 && (STEPW / 4) % 64 == 0 && (TAPW / 4) % 64 == 0, "tile shape");
  constexpr int WPT = (STEPW / 4 + kNT - 1) / kNT;  // float4 per thread per step (the last round: whole waves)
  const int XW = kTT + K - 1;
  const int XWP = (XW + 63) / 64 * 64;    // padded row: whole waves of the direct loads

  extern __shared__ float smem[];
  float* xs = smem;                       // [CPG][XWP]
  float* ws = smem + CPG * XWP;           // [2 buffers][kNQ parts][kKB][ci][co]

  const int g = blockIdx.y;
  const int b = blockIdx.z;
  const int t0 = blockIdx.x * kTT;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int half = wave >> 1;             // tap part
  const int sub = wave & 1;               // 16-column half of the tile
  const int kq = lane >> 4;
  const int l16 = lane & 15;

  const long long xrow0 = ((long long)b * H + (long long)g * CPG) * L;
  // the group's input rows (CPG * L floats) and its weights (K * TAPW)
  const __amdgpu_buffer_rsrc_t xrs = uniform_rsrc(x + xrow0, 4u * (unsigned)(CPG * L));
  const __amdgpu_buffer_rsrc_t wrs = uniform_rsrc(w + (long long)g * K * TAPW, 4u * (unsigned)(K * TAPW));

  // the input window: row ci, column j <-> x[ci][t0 - pad + j], 0 outside
  for (int f0 = 0; f0 < CPG * XWP; f0 += kNT) {
    const int f = f0 + tid;
    const int ci = f / XWP;
    const int j = f - ci * XWP;
    const int t = t0 - pad + j;
    const unsigned off = j < XW && t >= 0 && t < L ? 4u * (unsigned)(ci * L + t) : kBufOut;
    buffer_load_lds_b32(xrs, xs + f0 + wave * 64, off);
  }
  const int nstep = K / (kNQ * kKB);
  // staging step s: part h, tap kk of the step -> tap h * K / kNQ + s * kKB + kk
  auto stage = [&](int s, int nb) {
    float4* dst = reinterpret_cast<float4*>(ws + nb * STEPW);
#pragma unroll
    for (int e = 0; e < WPT; ++e) {
      if (e + 1 == WPT && e * kNT + wave * 64 >= STEPW / 4) break;  // wave-uniform
      const int f = e * kNT + tid;        // float4 of the step
      const int blk = f / (TAPW / 4);     // (part, kk)
      const int within = f - blk * (TAPW / 4);
      const int h = blk / kKB, kk = blk - h * kKB;
      const int tap = h * (K / kNQ) + s * kKB + kk;
      buffer_load_lds_b128(wrs, dst + e * kNT + wave * 64, 4u * (unsigned)(tap * TAPW + 4 * within));
    }
  };
  stage(0, 0);

  floatx4 acc[TM];
#pragma unroll
  for (int m = 0; m < TM; ++m) acc[m] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int col = sub * 16 + l16;         // this lane's column in the tile
  for (int s = 0; s < nstep; ++s) {
    __builtin_amdgcn_s_waitcnt(0);        // this wave's loads of step s (and the window) have landed
    __syncthreads();                      // ... and every wave's; step s - 1's buffer is free
    if (s + 1 < nstep) stage(s + 1, (s + 1) & 1);
    const float* wb = ws + (s & 1) * STEPW + half * kKB * TAPW;
#pragma unroll
    for (int kk = 0; kk < kKB; ++kk) {
      const int tap = half * (K / kNQ) + s * kKB + kk;
      const float* xk = xs + kq * XWP + col + tap;
      const float* wk = wb + kk * TAPW + kq * CPG + l16;
#pragma unroll
      for (int c = 0; c < CPG / 4; ++c) {
        const float bv = xk[4 * c * XWP];
#pragma unroll
        for (int m = 0; m < TM; ++m)
          acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(wk[4 * c * CPG + m * 16], bv, acc[m], 0, 0, 0);
      }
    }
  }
  // the other parts' sums to LDS (the weight buffers are free once every
  // wave passed the barrier), added to part 0's in part order
  __syncthreads();
  float* red = ws;                        // [part - 1][sub][m][r][lane]
  if (half > 0) {
#pragma unroll
    for (int m = 0; m < TM; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[((((half - 1) * 2 + sub) * TM + m) * 4 + r) * 64 + lane] = acc[m][r];
  }
  __syncthreads();
  if (half > 0) return;
  const int t = t0 + col;
  if (t >= L) return;
  float* ob = out + xrow0;
#pragma unroll
  for (int m = 0; m < TM; ++m)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int co = m * 16 + 4 * kq + r;
      float v = acc[m][r];
#pragma unroll
      for (int q = 1; q < kNQ; ++q) v = v + red[((((q - 1) * 2 + sub) * TM + m) * 4 + r) * 64 + lane];
      if (bias) v = v + bias[g * CPG + co];
      ob[(long long)co * L + t] = v;
    }
}

}  // namespace

bool posconv_supported(int cpg, int K, int pad) {
  return cpg == 48 && K >= kNQ * kKB && K % (kNQ * kKB) == 0 && pad >= 0 && pad < K;
}

void launch_posconv(const float* x, const float* w, const float* bias, float* out, int B, int H, int L, int cpg,
                    int K, int pad, hipStream_t s) {
  RVC_CHECK(posconv_supported(cpg, K, pad) && H % cpg == 0 && B >= 1 && L >= 1, "posconv: unsupported shape");
  RVC_CHECK(4LL * cpg * L < (1LL << 31) && 4LL * K * cpg * cpg < (1LL << 31), "posconv: tensors too large");
  const int XWP = (kTT + K - 1 + 63) / 64 * 64;
  const size_t lds = sizeof(float) * ((size_t)cpg * XWP + 2 * (size_t)kNQ * kKB * cpg * cpg);
  RVC_CHECK(lds <= 160 * 1024, "posconv: LDS above the CU's 160 KiB");
  static bool attr = false;
  if (!attr) {
    RVC_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&posconv_kernel<48>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
    attr = true;
  }
  const dim3 grid((unsigned)((L + kTT - 1) / kTT), (unsigned)(H / cpg), (unsigned)B);
  hipLaunchKernelGGL(posconv_kernel<48>, grid, dim3(kNT), lds, s, x, w, bias, out, H, L, K, pad);
  check_launch("posconv");
}

}  // namespace rvc
