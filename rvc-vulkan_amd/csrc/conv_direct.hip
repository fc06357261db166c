// Vector-ALU convolutions for the shapes the MFMA kernel does not cover:
//   * strided conv1d with few input channels (the NSF noise convs,
//     1 -> C with k = 2*stride; runtime/models/vits.py:1628-1635),
//   * conv_post (32 -> 1, k7, leaky 0.01 prologue, tanh epilogue;
//     runtime/models/vits.py:2228-2231) and other stride-1 launches with
//     fewer than 8 output channels, staged through LDS rows,
//   * the general op-level conv1d (stride > 1) and ConvTranspose1d with
//     dilation / output_padding (runtime/nn.py:89-135, 293-346).
// Plus the device-side weight packers for the MFMA kernel.
#include "internal.h"

namespace rvc {
namespace {

__device__ __forceinline__ float act_in(float v, int act, float slope) {
  return (act == ACT_LEAKY && v < 0.f) ? v * slope : v;
}

__device__ __forceinline__ float act_out(float v, int act, float slope) {
  if (act == ACT_LEAKY) return v >= 0.f ? v : v * slope;
  if (act == ACT_TANH) return tanhf(v);
  if (act == ACT_RELU) return fmaxf(v, 0.f);
  if (act == ACT_GELU) return gelu_as(v);
  return v;
}

// One thread per output position i, TCO output channels per workgroup: the
// weights are uniform across the workgroup (scalar loads) and each input
// sample is loaded once for all TCO channels.  Neighbouring threads' taps
// overlap, so the input reads are served by the L1/L2 caches.
template <int TCO>
__global__ __launch_bounds__(256) void conv1d_direct_kernel(DirectConvArgs a) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int co0 = blockIdx.y * TCO;
  const int b = blockIdx.z;
  if (i >= a.n_out) return;  // no barriers below
  const float* xb = a.x + (long long)b * a.xb;
  float acc[TCO];
#pragma unroll
  for (int c = 0; c < TCO; ++c) acc[c] = 0.f;
  const long long t0 = (long long)i * a.stride + a.in_off;
  for (int ci = 0; ci < a.C_in; ++ci) {
    const float* xr = xb + (long long)ci * a.xc;
    for (int k = 0; k < a.K; ++k) {
      const long long t = t0 + (long long)k * a.dil;
      const float v = (t >= 0 && t < a.L_in) ? act_in(xr[t], a.in_act, a.in_slope) : 0.f;
#pragma unroll
      for (int c = 0; c < TCO; ++c) {
        const int co = min(co0 + c, a.C_out - 1);
        acc[c] += a.w[((long long)co * a.C_in + ci) * a.K + k] * v;
      }
    }
  }
  float* ob = a.out + (long long)b * a.ob + i;
#pragma unroll
  for (int c = 0; c < TCO; ++c) {
    const int co = co0 + c;
    if (co >= a.C_out) break;
    float v = acc[c];
    if (a.bias) v = v + a.bias[co];
    v = act_out(v, a.out_act, a.out_slope);
    float* o = ob + (long long)co * a.oc;
    if (a.combine == COMB_ADD) v = *o + v;
    else if (a.combine == COMB_ADD_DIV) v = (*o + v) / a.div;
    *o = v;
  }
}

// Stride-1 convolution with few output channels (conv_post: 32 -> 1, k7):
// a workgroup owns 256 consecutive outputs of one output channel and walks
// the input channels kRowCh at a time, staging each channel's 256 + halo
// samples in LDS once (coalesced, input activation applied on the way in).
// Thread t computes output t, so a wave reads 64 neighbouring LDS words per
// tap; the small tile keeps several workgroups per CU in flight to hide the
// load latency of each chunk.  Per output the sum runs channel-major, taps
// inner, as in conv1d_direct_kernel.  With x2 / x3 the staged sample is the
// decoder's three-ResBlock average of the three inputs.
constexpr int kRowOut = 256, kRowCh = 8, kRowHaloMax = 128;
__global__ __launch_bounds__(256) void conv1d_rows_kernel(DirectConvArgs a) {
  __shared__ float rows[kRowCh][kRowOut + kRowHaloMax];
  const int i0 = blockIdx.x * kRowOut;
  const int co = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int W = kRowOut + (a.K - 1) * a.dil;  // launcher: (K - 1) * dil <= kRowHaloMax
  const float* xb = a.x + (long long)b * a.xb;
  const float* xb2 = a.x2 ? a.x2 + (long long)b * a.xb : nullptr;
  const float* xb3 = a.x2 ? a.x3 + (long long)b * a.xb : nullptr;
  const long long tb = (long long)i0 + a.in_off;
  float acc = 0.f;
  for (int ci0 = 0; ci0 < a.C_in; ci0 += kRowCh) {
    const int nch = min(kRowCh, a.C_in - ci0);
    for (int r = 0; r < nch; ++r) {
      const long long ro = (long long)(ci0 + r) * a.xc;
      for (int c = tid; c < W; c += 256) {
        const long long t = tb + c;
        float v = 0.f;
        if (t >= 0 && t < a.L_in) {
          v = xb[ro + t];
          if (xb2) v = div3_rn((v + xb2[ro + t]) + xb3[ro + t]);  // the decoder's ((o1 + o2) + o3) / 3
          v = act_in(v, a.in_act, a.in_slope);
        }
        rows[r][c] = v;
      }
    }
    __syncthreads();
    for (int r = 0; r < nch; ++r) {
      const float* wr = a.w + ((long long)co * a.C_in + ci0 + r) * a.K;
      for (int k = 0; k < a.K; ++k) {
        const float wv = wr[k];
        acc += wv * rows[r][tid + k * a.dil];
      }
    }
    __syncthreads();
  }
  float* ob = a.out + (long long)b * a.ob + (long long)co * a.oc;
  const int i = i0 + tid;
  if (i >= a.n_out) return;
  float v = acc;
  if (a.bias) v = v + a.bias[co];
  v = act_out(v, a.out_act, a.out_slope);
  float* o = ob + i;
  if (a.combine == COMB_ADD) v = *o + v;
  else if (a.combine == COMB_ADD_DIV) v = (*o + v) / a.div;
  *o = v;
}

// The decoder's conv_post (C_out = 1, stride 1, dilation 1, odd K <= 9 with
// "same" padding), HBM-bound: it streams every input channel once (with x2 /
// x3 the three ResBlock outputs of the last stage, averaged while staged).
// A workgroup owns kPostTile outputs, thread t outputs t0 + 4t .. + 3.  The
// channels go through LDS in groups of kPostCh: for each group every thread
// loads one aligned float4 of each channel row of each input (the first two
// threads also the 8-sample halo), forms ((x + x2) + x3) / 3 and the input
// activation, and stores the float4 to the group's LDS window
// [kPostCh][kPostTile + 8] (window column 0 = sample t0 - 4).  The next
// group's loads are issued before the current group's taps are summed, and
// the window is double-buffered, so one barrier per group remains.  Per
// output the sum runs channel-major, taps inner, like conv1d_rows_kernel.
// Requirements (checked by the launcher): L % 4 == 0 and 16-byte aligned
// rows, so each aligned float4 lies wholly inside [0, L) or wholly outside,
// and outside ones read 0 through the buffer range.
constexpr int kPostCh = 4;
template <int K, int NT, int CH>
__global__ __launch_bounds__(NT) void conv_post_kernel(DirectConvArgs a) {
  constexpr int kPostTile = 4 * NT, kPostW = kPostTile + 8;
  __shared__ float4 win[2][CH][kPostW / 4];
  const int tid = threadIdx.x;
  const int b = blockIdx.y;
  const int t0 = blockIdx.x * kPostTile;
  const int nin = a.x2 ? 3 : 1;
  const unsigned range = 4u * (unsigned)((a.C_in - 1) * (int)a.xc + a.L_in);
  const __amdgpu_buffer_rsrc_t r0 = uniform_rsrc(a.x + (long long)b * a.xb, range);
  const __amdgpu_buffer_rsrc_t r1 = uniform_rsrc(nin == 3 ? a.x2 + (long long)b * a.xb : a.x, range);
  const __amdgpu_buffer_rsrc_t r2 = uniform_rsrc(nin == 3 ? a.x3 + (long long)b * a.xb : a.x, range);
  // window float4 f covers samples t0 - 4 + 4f .. + 3: f = tid, and f = NT + tid for tid < 2
  auto foff = [&](int f, int c) -> unsigned {
    const int t = t0 - 4 + 4 * f;
    return (t >= 0 && t < a.L_in) ? 4u * (unsigned)(c * (int)a.xc + t) : kBufOut;
  };
  const bool halo = tid < 2;
  float4 v[3][CH], h[3][CH];
  auto load = [&](int c0) {
#pragma unroll
    for (int r = 0; r < CH; ++r) {
      const unsigned o = foff(tid, c0 + r);
      const unsigned oh = halo ? foff(NT + tid, c0 + r) : kBufOut;
      v[0][r] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r0, o, 0, 0));
      if (halo) h[0][r] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r0, oh, 0, 0));
      if (nin == 3) {
        v[1][r] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r1, o, 0, 0));
        v[2][r] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r2, o, 0, 0));
        if (halo) {
          h[1][r] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r1, oh, 0, 0));
          h[2][r] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r2, oh, 0, 0));
        }
      }
    }
  };
  auto prep = [&](float4 x, float4 y, float4 z) -> float4 {
    float e[4] = {x.x, x.y, x.z, x.w};
    if (nin == 3) {
      const float f[4] = {y.x, y.y, y.z, y.w}, g[4] = {z.x, z.y, z.z, z.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) e[i] = div3_rn((e[i] + f[i]) + g[i]);  // the decoder's ((o1 + o2) + o3) / 3
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) e[i] = act_in(e[i], a.in_act, a.in_slope);
    return float4{e[0], e[1], e[2], e[3]};
  };
  constexpr int c_off = 4 - (K - 1) / 2;  // window column of output 4t's first tap, minus 4t
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  const int ng = a.C_in / CH;
  load(0);
  for (int g = 0; g < ng; ++g) {
    const int buf = g & 1;
#pragma unroll
    for (int r = 0; r < CH; ++r) {
      win[buf][r][tid] = prep(v[0][r], v[1][r], v[2][r]);
      if (halo) win[buf][r][NT + tid] = prep(h[0][r], h[1][r], h[2][r]);
    }
    __syncthreads();
    if (g + 1 < ng) load((g + 1) * CH);
#pragma unroll
    for (int r = 0; r < CH; ++r) {
      const float* wl = reinterpret_cast<const float*>(&win[buf][r][0]) + 4 * tid + c_off;
      float x[K + 3];
#pragma unroll
      for (int i = 0; i < K + 3; ++i) x[i] = wl[i];
      const float* wr = a.w + (long long)(g * CH + r) * K;
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const float wv = wr[k];
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[q] += wv * x[q + k];
      }
    }
  }
  const int o0 = t0 + 4 * tid;
  if (o0 >= a.n_out) return;
  float res[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float u = acc[q];
    if (a.bias) u = u + a.bias[0];
    res[q] = act_out(u, a.out_act, a.out_slope);
  }
  float* ob = a.out + (long long)b * a.ob + o0;
  *reinterpret_cast<float4*>(ob) = float4{res[0], res[1], res[2], res[3]};
}

bool conv_post_ok(const DirectConvArgs& a) {
  return a.C_out == 1 && a.stride == 1 && a.dil == 1 && a.K % 2 == 1 && a.K >= 3 && a.K <= 9 && a.in_off == -(a.K - 1) / 2 &&
         a.n_out == a.L_in && a.L_in % 4 == 0 && a.C_in % kPostCh == 0 && a.xc % 4 == 0 && a.xb % 4 == 0 &&
         a.ob % 4 == 0 && a.combine == COMB_STORE && (reinterpret_cast<uintptr_t>(a.out) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 && (!a.x2 || ((reinterpret_cast<uintptr_t>(a.x2) & 15) == 0 &&
                                                            (reinterpret_cast<uintptr_t>(a.x3) & 15) == 0)) &&
         4.0 * ((a.C_in - 1) * (double)a.xc + a.L_in) < 2147483648.0;
}

// Single-input-channel convolutions at dilation 1 (the NSF noise convs of
// the decoder stages the ConvTranspose epilogue does not cover: 1 -> C with
// k = 2 * stride, runtime/models/vits.py:1628-1635).  A workgroup owns
// kC1Out outputs x kC1Co channels.  The input window is staged phase-major,
// xs[r][m] = x[t0 + m * stride + r], so output j's tap k reads
// xs[k % stride][j + k / stride] and a wave's 32 neighbouring outputs read
// 32 consecutive LDS words; the weights are staged [k][32 channels] and read
// as float4 broadcasts.  Thread t forms outputs t % 32 + 32u (u < 4) of
// channels 4 * (t / 32) .. +3, the taps summed in order.
constexpr int kC1Out = 128, kC1Co = 32;
size_t c1_lds_floats(int K, int stride) {
  const int M = kC1Out + (K - 1) / stride + 1;
  return (size_t)K * kC1Co + (size_t)stride * M;
}
__global__ __launch_bounds__(256) void conv1d_c1_kernel(DirectConvArgs a) {
  extern __shared__ float sm[];
  const int i0 = blockIdx.x * kC1Out, co0 = blockIdx.y * kC1Co, b = blockIdx.z;
  const int S = a.stride, K = a.K;
  const int M = kC1Out + (K - 1) / S + 1;  // columns per phase row
  float* ws = sm;                          // [K][kC1Co]
  float* xs = sm + K * kC1Co;              // [S][M]
  const int tid = threadIdx.x;
  for (int e = tid; e < K * kC1Co; e += 256) {
    const int k = e / kC1Co, c = e - k * kC1Co;
    const int co = co0 + c;
    ws[e] = co < a.C_out ? a.w[(long long)co * K + k] : 0.f;
  }
  const float* xb = a.x + (long long)b * a.xb;
  const long long tb = (long long)i0 * S + a.in_off;
  for (int q = tid; q < S * M; q += 256) {  // global order: coalesced reads
    const int m = q / S, r = q - m * S;
    const long long t = tb + q;
    xs[r * M + m] = (t >= 0 && t < a.L_in) ? act_in(xb[t], a.in_act, a.in_slope) : 0.f;
  }
  __syncthreads();
  const int jl = tid & 31, cq = tid >> 5;
  float acc[4][4];
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[u][c] = 0.f;
  for (int k = 0; k < K; ++k) {
    const float4 wv = *reinterpret_cast<const float4*>(ws + k * kC1Co + 4 * cq);
    const float* xr = xs + (k % S) * M + k / S + jl;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float xv = xr[32 * u];
      acc[u][0] += wv.x * xv;
      acc[u][1] += wv.y * xv;
      acc[u][2] += wv.z * xv;
      acc[u][3] += wv.w * xv;
    }
  }
  float* ob = a.out + (long long)b * a.ob;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int co = co0 + 4 * cq + c;
    if (co >= a.C_out) break;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + jl + 32 * u;
      if (i >= a.n_out) continue;
      float v = acc[u][c];
      if (a.bias) v = v + a.bias[co];
      v = act_out(v, a.out_act, a.out_slope);
      float* o = ob + (long long)co * a.oc + i;
      if (a.combine == COMB_ADD) v = *o + v;
      else if (a.combine == COMB_ADD_DIV) v = (*o + v) / a.div;
      *o = v;
    }
  }
}

// Gather-form ConvTranspose1d: one thread per output element.
__global__ __launch_bounds__(256) void conv_t1d_direct_kernel(ConvTArgs a) {
  const long long n = (long long)a.B * a.C_out * a.n_out;
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n) return;
  const int o = (int)(idx % a.n_out);
  const int co = (int)((idx / a.n_out) % a.C_out);
  const int b = (int)(idx / ((long long)a.n_out * a.C_out));
  const float* xb = a.x + (long long)b * a.xb;
  const int lo = a.win_len > 0 ? max(a.win_lo, 0) : 0;
  const int hi = a.win_len > 0 ? min(a.win_lo + a.win_len, a.L_in) : a.L_in;
  float acc = 0.f;
  for (int k = 0; k < a.K; ++k) {
    const int num = o + a.o_off + a.padding - k * a.dil;
    if (num < 0 || num % a.stride != 0) continue;
    const int t = num / a.stride;
    if (t < lo || t >= hi) continue;
    for (int ci = 0; ci < a.C_in; ++ci)
      acc += act_in(xb[(long long)ci * a.xc + t], a.in_act, a.in_slope) *
             a.w[((long long)ci * a.C_out + co) * a.K + k];
  }
  float v = acc;
  if (a.bias) v = v + a.bias[co];
  float* out = a.out + (long long)b * a.ob + (long long)co * a.oc + o + a.o_off;
  if (a.combine == COMB_ADD) v = *out + v;
  *out = v;
}

// idx enumerates the destination [K][C_in][ld]; columns co >= C_out are zero
__global__ void pack_conv_weight_kernel(const float* w, float* out, int C_out, int C_in, int K, int ld) {
  const long long n = (long long)ld * C_in * K;
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n) return;
  const int co = (int)(idx % ld);
  const int ci = (int)((idx / ld) % C_in);
  const int k = (int)(idx / ((long long)ld * C_in));
  out[idx] = co < C_out ? w[((long long)co * C_in + ci) * K + k] : 0.f;
}

__global__ void pack_convt_phase_kernel(const float* w, float* out, int C_in, int C_out, int K, int st,
                                        int r, int J, int ld) {
  const long long n = (long long)J * C_in * ld;
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n) return;
  const int co = (int)(idx % ld);
  const int ci = (int)((idx / ld) % C_in);
  const int jp = (int)(idx / ((long long)ld * C_in));
  const int k = r + (J - 1 - jp) * st;
  out[idx] = co < C_out ? w[((long long)ci * C_out + co) * K + k] : 0.f;
}

__device__ __forceinline__ uint16_t bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// [C_out][C_in][K] fp32 -> [K][C_out][ldi] bf16; idx enumerates the destination
__global__ void pack_conv_weight_bf16_kernel(const float* w, uint16_t* out, int C_out, int C_in, int K, int ldi) {
  const long long n = (long long)K * C_out * ldi;
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n) return;
  const int ci = (int)(idx % ldi);
  const int co = (int)((idx / ldi) % C_out);
  const int k = (int)(idx / ((long long)ldi * C_out));
  out[idx] = ci < C_in ? bf16_rne(w[((long long)co * C_in + ci) * K + k]) : (uint16_t)0;
}

// phase r of a ConvTranspose1d, [C_in][C_out][K] fp32 -> [J][C_out][ldi] bf16
__global__ void pack_convt_phase_bf16_kernel(const float* w, uint16_t* out, int C_in, int C_out, int K, int st,
                                             int r, int J, int ldi) {
  const long long n = (long long)J * C_out * ldi;
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n) return;
  const int ci = (int)(idx % ldi);
  const int co = (int)((idx / ldi) % C_out);
  const int jp = (int)(idx / ((long long)ldi * C_out));
  const int k = r + (J - 1 - jp) * st;
  out[idx] = ci < C_in ? bf16_rne(w[((long long)ci * C_out + co) * K + k]) : (uint16_t)0;
}

unsigned grid1d(long long n) { return (unsigned)((n + 255) / 256); }

}  // namespace

void launch_conv1d_direct(const DirectConvArgs& a, hipStream_t s) {
  RVC_CHECK(a.C_in >= 1 && a.C_out >= 1 && a.K >= 1 && a.stride >= 1 && a.dil >= 1 && a.B >= 1,
            "conv1d_direct: invalid shape");
  RVC_CHECK(!a.x2 || (a.x3 && a.C_out < 8 && a.stride == 1 && (long long)(a.K - 1) * a.dil <= kRowHaloMax),
            "conv1d_direct: a three-input average needs the stride-1 row kernel");
  if (a.n_out <= 0) return;
  if (a.C_in == 1 && a.dil == 1 && !a.x2 && a.C_out >= 8 && a.stride <= 64 &&
      c1_lds_floats(a.K, a.stride) * sizeof(float) <= 65536) {
    dim3 grid((a.n_out + kC1Out - 1) / kC1Out, (a.C_out + kC1Co - 1) / kC1Co, a.B);
    launch_timed(conv1d_c1_kernel, grid, dim3(256), c1_lds_floats(a.K, a.stride) * sizeof(float), s, a);
  } else if (a.C_out >= 8) {
    dim3 grid((a.n_out + 255) / 256, (a.C_out + 7) / 8, a.B);
    hipLaunchKernelGGL(conv1d_direct_kernel<8>, grid, dim3(256), 0, s, a);
  } else if (conv_post_ok(a)) {
    constexpr int NT = 256, CH = kPostCh;
    dim3 grid((a.n_out + 4 * NT - 1) / (4 * NT), a.B);
    switch (a.K) {
      case 3: launch_timed(conv_post_kernel<3, NT, CH>, grid, dim3(NT), 0, s, a); break;
      case 5: launch_timed(conv_post_kernel<5, NT, CH>, grid, dim3(NT), 0, s, a); break;
      case 7: launch_timed(conv_post_kernel<7, NT, CH>, grid, dim3(NT), 0, s, a); break;
      default: launch_timed(conv_post_kernel<9, NT, CH>, grid, dim3(NT), 0, s, a); break;
    }
  } else if (a.stride == 1 && (long long)(a.K - 1) * a.dil <= kRowHaloMax) {
    dim3 grid((a.n_out + kRowOut - 1) / kRowOut, a.C_out, a.B);
    hipLaunchKernelGGL(conv1d_rows_kernel, grid, dim3(256), 0, s, a);
  } else {
    dim3 grid((a.n_out + 255) / 256, a.C_out, a.B);
    hipLaunchKernelGGL(conv1d_direct_kernel<1>, grid, dim3(256), 0, s, a);
  }
  check_launch("conv1d_direct");
}

void launch_conv_t1d_direct(const ConvTArgs& a, hipStream_t s) {
  RVC_CHECK(a.C_in >= 1 && a.C_out >= 1 && a.K >= 1 && a.stride >= 1 && a.dil >= 1 && a.B >= 1,
            "conv_t1d_direct: invalid shape");
  const long long n = (long long)a.B * a.C_out * a.n_out;
  if (n <= 0) return;
  hipLaunchKernelGGL(conv_t1d_direct_kernel, dim3(grid1d(n)), dim3(256), 0, s, a);
  check_launch("conv_t1d_direct");
}

void launch_pack_conv_weight(const float* w, float* out, int C_out, int C_in, int K, hipStream_t s) {
  const int ld = packed_ld(C_out);
  const long long n = (long long)ld * C_in * K;
  if (n == 0) return;
  hipLaunchKernelGGL(pack_conv_weight_kernel, dim3(grid1d(n)), dim3(256), 0, s, w, out, C_out, C_in, K, ld);
  check_launch("pack_conv_weight");
}

void launch_pack_convt_phase(const float* w, float* out, int C_in, int C_out, int K, int st, int r,
                             int J, hipStream_t s) {
  const int ld = packed_ld(C_out);
  const long long n = (long long)J * C_in * ld;
  if (n == 0) return;
  hipLaunchKernelGGL(pack_convt_phase_kernel, dim3(grid1d(n)), dim3(256), 0, s, w, out, C_in, C_out, K,
                     st, r, J, ld);
  check_launch("pack_convt_phase");
}

void launch_pack_conv_weight_bf16(const float* w, uint16_t* out, int C_out, int C_in, int K, hipStream_t s) {
  const int ldi = bf16_ld(C_in);
  const long long n = (long long)K * C_out * ldi;
  if (n == 0) return;
  hipLaunchKernelGGL(pack_conv_weight_bf16_kernel, dim3(grid1d(n)), dim3(256), 0, s, w, out, C_out, C_in, K, ldi);
  check_launch("pack_conv_weight_bf16");
}

void launch_pack_convt_phase_bf16(const float* w, uint16_t* out, int C_in, int C_out, int K, int st, int r, int J,
                                  hipStream_t s) {
  const int ldi = bf16_ld(C_in);
  const long long n = (long long)J * C_out * ldi;
  if (n == 0) return;
  hipLaunchKernelGGL(pack_convt_phase_bf16_kernel, dim3(grid1d(n)), dim3(256), 0, s, w, out, C_in, C_out, K, st, r, J,
                     ldi);
  check_launch("pack_convt_phase_bf16");
}

}  // namespace rvc
