// RMVPE pitch extraction kernels for gfx950: the 2-D convolutions of the
// U-Net on fp32 matrix cores, the mel front end's framing / magnitude / log,
// 2x2 average pooling, the bidirectional GRU recurrence and the
// local-average cents decode.
//
// conv2d: implicit GEMM with M = C_out, N = computed points, reduction over
// (tap, input channel), on v_mfma_f32_16x16x4_f32 (16-row tiles suit the 16-
// and 32-channel U-Net levels).  A workgroup owns BM output channels x BN
// points laid out as TR rows x TC columns of the computed grid (TC = BN when
// the grid is wide, a narrower power of two for the deep levels whose rows
// hold 4..64 points).  Per chunk of BK input channels it stages in LDS the
// input window those points read -- (TR-1)*S + 1 + span rows by (TC-1)*S + 1
// + span columns, zero outside the image -- once for all taps, plus the
// packed weights [tap][BK][BM].  Lane l of an MFMA step supplies
//   A = W[t][c + l/16][co_tile + l%16]
//   B = xs[c + l/16][point(l%16) + tap offset]
// and its 4 accumulators hold rows 4*(l/16) + r, column l%16.  Groups of one
// launch (grid z) are independent convolutions sharing the channel counts:
// the four phases of a stride-2 ConvTranspose2d.  Few computed points (the
// deep levels: 128..2048 points for 256..512 channels) split the channels
// over workgroups; a deterministic reduce adds the partial sums in order and
// applies the epilogue.
#include <algorithm>
#include <cmath>

#include "internal.h"

namespace rvc {

typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

template <int BN, int S>
constexpr int conv2d_window_max() {
  // largest (TR-1)*S+3 by (TC-1)*S+3 window over TR*TC = BN, spans <= 2
  return 3 * ((BN - 1) * S + 3);
}

template <int BM, int BN, int WM, int WN, int BK, int S>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void conv2d_mfma_kernel(Conv2dLaunch a) {
  constexpr int NWM = BM / WM, NWN = BN / WN;
  constexpr int NT = NWM * NWN * 64;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int XPT = (BK * conv2d_window_max<BN, S>() + NT - 1) / NT;
  constexpr int W4 = BM / 4;
  constexpr int WPT = (kConv2dTapsMax * BK * W4 + NT - 1) / NT;
  static_assert(BK % 4 == 0 && BM % 16 == 0 && WM % 16 == 0 && WN % 16 == 0, "tile shape");

  const int nz = a.n_groups * a.B;
  const int z = blockIdx.z % nz;
  const int ks = blockIdx.z / nz;
  const int gi = z / a.B;
  const int bb = z - gi * a.B;
  const Conv2dGroup& G = a.g[gi];
  const int TC = a.tile_c;
  const int TR = BN / TC;
  const int ntc = (a.OW + TC - 1) / TC;
  const int tr = blockIdx.x / ntc;
  const int a0 = tr * TR;
  const int b0 = (blockIdx.x - tr * ntc) * TC;
  const int co0 = blockIdx.y * BM;
  const int WR = (TR - 1) * S + 1 + G.dh_span;
  const int WC = (TC - 1) * S + 1 + G.dw_span;
  const int plane = WR * WC;
  const int xfl = (BK * plane + 3) / 4 * 4;  // weights start 16-byte aligned
  const int h_lo = a0 * S + G.dh_lo;
  const int w_lo = b0 * S + G.dw_lo;
  const int csplit = a.ksplit > 1 ? a.csplit : a.C_in;
  const int ci_lo = ks * csplit;
  const int ci_hi = min(a.C_in, ci_lo + csplit);
  const int T = G.ntaps;

  extern __shared__ float smem[];
  float* xs = smem;
  float* ws = smem + xfl;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % NWM;
  const int wn = wave / NWM;
  const int kq = lane >> 4;
  const int l16 = lane & 15;

  // staging map (fixed across chunks): input element e -> channel row and
  // offset within that channel's plane (-1: outside the image / window).
  // The quotients by the runtime plane / row widths come from a float
  // reciprocal and one correction step (exact: operands < 2^24).
  const int nx = BK * plane;
  const float inv_plane = 1.0f / (float)plane;
  const float inv_wc = 1.0f / (float)WC;
  auto qdiv = [](int n, int d, float inv) {
    int q = (int)((float)n * inv);
    if (q * d > n) --q;
    else if ((q + 1) * d <= n) ++q;
    return q;
  };
  int xo[XPT], xr[XPT];
#pragma unroll
  for (int e = 0; e < XPT; ++e) {
    const int idx = tid + e * NT;
    const int r = qdiv(idx, plane, inv_plane);
    const int rem = idx - r * plane;
    const int rr = qdiv(rem, WC, inv_wc);
    const int cc = rem - rr * WC;
    const int h = h_lo + rr;
    const int w = w_lo + cc;
    const bool ok = idx < nx && h >= 0 && h < a.H && w >= 0 && w < a.W;
    xr[e] = idx < nx ? r : -1;
    xo[e] = ok ? h * a.W + w : -1;
  }
  const int nw4 = T * BK * W4;
  int wo[WPT], wc[WPT];
#pragma unroll
  for (int e = 0; e < WPT; ++e) {
    const int idx = tid + e * NT;
    const int row = idx / W4;
    const int c4 = idx - row * W4;
    const int t = row / BK;
    const int c = row - t * BK;
    const bool ok = idx < nw4 && co0 + 4 * c4 < a.w_ld;
    wc[e] = idx < nw4 ? (ok ? c : 1 << 20) : -1;
    wo[e] = ok ? (t * a.C_in + c) * a.w_ld + co0 + 4 * c4 : 0;
  }

  const float* xbat = a.x + (long long)bb * a.xb;
  float xv[XPT];
  float4 wv[WPT];
  auto gload = [&](int ci0) {
    const float* xc0 = xbat + (long long)ci0 * a.xc;
    const float* wc0 = G.w + (long long)ci0 * a.w_ld;
    const int lim = ci_hi - ci0;
#pragma unroll
    for (int e = 0; e < XPT; ++e)
      xv[e] = (xo[e] >= 0 && xr[e] < lim) ? xc0[(long long)xr[e] * a.xc + xo[e]] : 0.f;
#pragma unroll
    for (int e = 0; e < WPT; ++e)
      wv[e] = (wc[e] >= 0 && wc[e] < lim) ? *reinterpret_cast<const float4*>(wc0 + wo[e])
                                           : make_float4(0.f, 0.f, 0.f, 0.f);
  };
  auto lstore = [&]() {
#pragma unroll
    for (int e = 0; e < XPT; ++e)
      if (xr[e] >= 0) xs[tid + e * NT] = xv[e];
#pragma unroll
    for (int e = 0; e < WPT; ++e)
      if (wc[e] >= 0) reinterpret_cast<float4*>(ws)[tid + e * NT] = wv[e];
  };

  floatx4 acc[TM][TN];
#pragma unroll
  for (int m = 0; m < TM; ++m)
#pragma unroll
    for (int n = 0; n < TN; ++n) acc[m][n] = floatx4{0.f, 0.f, 0.f, 0.f};

  // LDS offset of the window corner each of this lane's points reads (TC is
  // a power of two)
  const int tcs = __builtin_ctz(TC);
  int pb[TN];
#pragma unroll
  for (int n = 0; n < TN; ++n) {
    const int pn = wn * WN + n * 16 + l16;
    const int pr = pn >> tcs;
    const int pc = pn & (TC - 1);
    pb[n] = pr * S * WC + pc * S;
  }

  if (ci_hi > ci_lo && T > 0) {
    const int nchunk = (ci_hi - ci_lo + BK - 1) / BK;
    gload(ci_lo);
    for (int c = 0; c < nchunk; ++c) {
      __syncthreads();  // every wave is done reading the previous chunk
      lstore();
      __syncthreads();
      if (c + 1 < nchunk) gload(ci_lo + (c + 1) * BK);  // in flight during the MFMAs
      const float* wbase = ws + kq * BM + wm * WM + l16;
      const float* xbase = xs + kq * plane;
      for (int t = 0; t < T; ++t) {
        const int toff = (G.dh[t] - G.dh_lo) * WC + (G.dw[t] - G.dw_lo);
#pragma unroll
        for (int q = 0; q < BK / 4; ++q) {
          float av[TM], bv[TN];
          const float* w_ = wbase + (t * BK + 4 * q) * BM;
          const float* x_ = xbase + 4 * q * plane + toff;
#pragma unroll
          for (int m = 0; m < TM; ++m) av[m] = w_[m * 16];
#pragma unroll
          for (int n = 0; n < TN; ++n) bv[n] = x_[pb[n]];
#pragma unroll
          for (int m = 0; m < TM; ++m)
#pragma unroll
            for (int n = 0; n < TN; ++n)
              acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[m], bv[n], acc[m][n], 0, 0, 0);
        }
      }
    }
  }

  // epilogue
  const long long npix = (long long)a.OH * a.OW;
  float* ob = a.out + (long long)bb * a.ob;
  const float* rb = a.res ? a.res + (long long)bb * a.ob : nullptr;
#pragma unroll
  for (int m = 0; m < TM; ++m)
#pragma unroll
    for (int n = 0; n < TN; ++n) {
      const int pn = wn * WN + n * 16 + l16;
      const int pa = a0 + (pn >> tcs);
      const int pw = b0 + (pn & (TC - 1));
      if (pa >= G.oh_n || pw >= G.ow_n) continue;
      const bool taps = pa < G.a_lim && pw < G.b_lim;
      const long long o = (long long)(pa * a.osh + G.oh0) * a.ors + (long long)(pw * a.osw + G.ow0) * a.ocs;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int co = co0 + wm * WM + m * 16 + 4 * kq + r;
        if (co >= a.C_out) continue;
        const float s = taps ? acc[m][n][r] : 0.f;
        if (a.ksplit > 1) {
          a.part[((long long)(ks * nz + z) * a.C_out + co) * npix + (long long)pa * a.OW + pw] = s;
          continue;
        }
        float v = s;
        if (a.bias) v = v + a.bias[co];
        if (a.relu) v = fmaxf(v, 0.f);
        if (rb) v = v + rb[co * a.oc + o];
        ob[co * a.oc + o] = v;
      }
    }
}

__global__ __launch_bounds__(256) void conv2d_reduce_kernel(Conv2dLaunch a) {
  const int nz = a.n_groups * a.B;
  const long long npix = (long long)a.OH * a.OW;
  const long long total = (long long)nz * a.C_out * npix;
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const long long p = idx % npix;
  const int co = (int)((idx / npix) % a.C_out);
  const int z = (int)(idx / (npix * a.C_out));
  const int gi = z / a.B;
  const int bb = z - gi * a.B;
  // the splits' partial sums in split order, kU loads in flight together
  constexpr int kU = 8;
  const long long kstride = (long long)nz * a.C_out * npix;
  const float* pp = a.part + ((long long)z * a.C_out + co) * npix + p;
  float s = 0.f;
  for (int k0 = 0; k0 < a.ksplit; k0 += kU) {
    float v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) v[u] = pp[min(k0 + u, a.ksplit - 1) * kstride];  // past ksplit: skipped below
#pragma unroll
    for (int u = 0; u < kU; ++u)
      if (k0 + u < a.ksplit) s += v[u];
  }
  const int pa = (int)(p / a.OW);
  const int pw = (int)(p - (long long)pa * a.OW);
  const Conv2dGroup& G = a.g[gi];
  if (pa >= G.oh_n || pw >= G.ow_n) return;
  const long long o = (long long)(pa * a.osh + G.oh0) * a.ors + (long long)(pw * a.osw + G.ow0) * a.ocs;
  float v = s;
  if (a.bias) v = v + a.bias[co];
  if (a.relu) v = fmaxf(v, 0.f);
  const long long oo = (long long)bb * a.ob + co * a.oc + o;
  if (a.res) v = v + a.res[oo];
  a.out[oo] = v;
}

struct Conv2dCfg {
  int BM, BN;
};

template <int BM, int BN, int WM, int WN, int BK, int S>
void run_conv2d(const Conv2dLaunch& a, int n_tiles, int n_co, int nz, hipStream_t st) {
  int maxplane = 0, maxt = 0;
  const int TC = a.tile_c, TR = BN / TC;
  for (int g = 0; g < a.n_groups; ++g) {
    const int wr = (TR - 1) * S + 1 + a.g[g].dh_span, wc = (TC - 1) * S + 1 + a.g[g].dw_span;
    maxplane = std::max(maxplane, wr * wc);
    maxt = std::max(maxt, a.g[g].ntaps);
    RVC_CHECK((wr * wc <= conv2d_window_max<BN, S>()), "conv2d: staged window exceeds the tile bound");
  }
  const size_t lds = sizeof(float) * ((size_t)(BK * maxplane + 3) / 4 * 4 + (size_t)maxt * BK * BM);
  RVC_CHECK(lds <= 65536, "conv2d: LDS budget exceeded");
  dim3 grid(n_tiles, n_co, nz * std::max(1, a.ksplit));
  hipLaunchKernelGGL((conv2d_mfma_kernel<BM, BN, WM, WN, BK, S>), grid, dim3((BM / WM) * (BN / WN) * 64), lds, st, a);
  check_launch("conv2d_mfma");
}

int pow2_at_least(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

long long conv2d_tiles(const Conv2dLaunch& a, const Conv2dCfg& c) {
  const int tc = std::min(c.BN, pow2_at_least(a.OW));
  const int tr = c.BN / tc;
  return (long long)((a.OH + tr - 1) / tr) * ((a.OW + tc - 1) / tc) * ((a.C_out + c.BM - 1) / c.BM) * a.n_groups *
         a.B;
}

// Largest tile whose grid gives every CU about four workgroups (256 CUs):
// each launch is short (0.6 GFLOP per U-Net conv at 10 s), so resident
// workgroups hide one another's load latency; 16-row tiles for 16 output
// channels.  When even 32 x 32 tiles leave CUs idle, the channels are split
// over workgroups (conv2d_plan).
constexpr long long kConv2dWant = 1024;
Conv2dCfg conv2d_cfg(const Conv2dLaunch& a) {
  if (a.stride == 2) return {32, 64};
  if (a.C_out <= 16) return conv2d_tiles(a, {16, 256}) >= kConv2dWant ? Conv2dCfg{16, 256} : Conv2dCfg{16, 128};
  static const Conv2dCfg order[] = {{64, 128}, {32, 128}, {64, 64}, {32, 64}, {32, 32}};
  for (const Conv2dCfg& c : order) {
    if (c.BM == 64 && a.C_out <= 32) continue;
    if (conv2d_tiles(a, c) >= kConv2dWant) return c;
  }
  return {32, 32};
}

// channel split over workgroups when the tile grid cannot fill the GPU:
// about kConv2dWant workgroups, at least 4 chunks of 8 channels per split
void conv2d_plan(Conv2dLaunch& a, const Conv2dCfg& c, int& n_tiles, int& n_co, int& nz) {
  a.tile_c = std::min(c.BN, pow2_at_least(a.OW));
  const int TR = c.BN / a.tile_c;
  n_tiles = ((a.OH + TR - 1) / TR) * ((a.OW + a.tile_c - 1) / a.tile_c);
  n_co = (a.C_out + c.BM - 1) / c.BM;
  nz = a.n_groups * a.B;
  a.ksplit = 1;
  a.csplit = a.C_in;
  const long long tiles = (long long)n_tiles * n_co * nz;
  const int BK = 8, min_ch = 4 * BK;
  if (tiles < 256 && a.C_in >= 2 * min_ch) {
    int ks = (int)std::min<long long>((kConv2dWant + tiles - 1) / tiles, a.C_in / min_ch);
    int cs = ((a.C_in + ks - 1) / ks + BK - 1) / BK * BK;
    ks = (a.C_in + cs - 1) / cs;
    if (ks > 1) {
      a.ksplit = ks;
      a.csplit = cs;
    }
  }
}

}  // namespace

size_t conv2d_split_floats(const Conv2dLaunch& a0) {
  Conv2dLaunch a = a0;
  int n_tiles, n_co, nz;
  conv2d_plan(a, conv2d_cfg(a), n_tiles, n_co, nz);
  return a.ksplit > 1 ? (size_t)a.ksplit * nz * a.C_out * a.OH * a.OW : 0;
}

void launch_conv2d(const Conv2dLaunch& a0, hipStream_t st) {
  Conv2dLaunch a = a0;
  RVC_CHECK(a.n_groups >= 1 && a.n_groups <= kConv2dGroupsMax, "conv2d: bad group count");
  RVC_CHECK(a.C_in >= 1 && a.C_out >= 1 && a.B >= 1 && a.H >= 1 && a.W >= 1 && a.w_ld >= a.C_out &&
                a.w_ld % 4 == 0, "conv2d: invalid shape");
  RVC_CHECK(a.stride == 1 || a.stride == 2, "conv2d: stride must be 1 or 2");
  RVC_CHECK(a.OH >= 0 && a.OW >= 0, "conv2d: negative output extent");
  if (a.OH == 0 || a.OW == 0) return;
  RVC_CHECK((long long)a.H * a.W < (1LL << 31) && (long long)a.OH * a.OW < (1LL << 31) &&
                (long long)8 * a.H * a.W < (1LL << 31), "conv2d: plane too large");
  for (int g = 0; g < a.n_groups; ++g) {
    Conv2dGroup& G = a.g[g];
    RVC_CHECK(G.ntaps >= 1 && G.ntaps <= kConv2dTapsMax, "conv2d: 1..9 taps per group");
    RVC_CHECK((reinterpret_cast<uintptr_t>(G.w) & 15) == 0, "conv2d: weights must be 16-byte aligned");
    int hl = G.dh[0], hh = G.dh[0], wl = G.dw[0], wh = G.dw[0];
    for (int t = 1; t < G.ntaps; ++t) {
      hl = std::min(hl, G.dh[t]); hh = std::max(hh, G.dh[t]);
      wl = std::min(wl, G.dw[t]); wh = std::max(wh, G.dw[t]);
    }
    RVC_CHECK(hh - hl <= 2 && wh - wl <= 2, "conv2d: tap offsets must span at most 3 rows and 3 columns");
    RVC_CHECK(G.oh_n >= 0 && G.oh_n <= a.OH && G.ow_n >= 0 && G.ow_n <= a.OW, "conv2d: group extent outside the grid");
    G.dh_lo = hl; G.dw_lo = wl; G.dh_span = hh - hl; G.dw_span = wh - wl;
  }
  const Conv2dCfg c = conv2d_cfg(a);
  int n_tiles, n_co, nz;
  conv2d_plan(a, c, n_tiles, n_co, nz);
  if (a.ksplit > 1 && (!a.part || a.part_floats < (size_t)a.ksplit * nz * a.C_out * a.OH * a.OW)) {
    a.ksplit = 1;
    a.csplit = a.C_in;
  }
  if (a.stride == 2)
    run_conv2d<32, 64, 32, 16, 8, 2>(a, n_tiles, n_co, nz, st);
  else if (c.BM == 16 && c.BN == 256)
    run_conv2d<16, 256, 16, 64, 8, 1>(a, n_tiles, n_co, nz, st);
  else if (c.BM == 16)
    run_conv2d<16, 128, 16, 32, 8, 1>(a, n_tiles, n_co, nz, st);
  else if (c.BM == 64 && c.BN == 128)
    run_conv2d<64, 128, 32, 64, 8, 1>(a, n_tiles, n_co, nz, st);
  else if (c.BM == 32 && c.BN == 128)
    run_conv2d<32, 128, 32, 32, 8, 1>(a, n_tiles, n_co, nz, st);
  else if (c.BM == 64 && c.BN == 64)
    run_conv2d<64, 64, 32, 32, 8, 1>(a, n_tiles, n_co, nz, st);
  else if (c.BN == 64)
    run_conv2d<32, 64, 16, 32, 8, 1>(a, n_tiles, n_co, nz, st);
  else
    run_conv2d<32, 32, 16, 16, 8, 1>(a, n_tiles, n_co, nz, st);
  if (a.ksplit > 1) {
    const long long total = (long long)nz * a.C_out * a.OH * a.OW;
    hipLaunchKernelGGL(conv2d_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, a);
    check_launch("conv2d_reduce");
  }
}

std::vector<float> pack_conv2d_host(const float* w, const float* scale, int C_out, int C_in, int KH, int KW) {
  const int ld = packed_ld(C_out);
  std::vector<float> o((size_t)KH * KW * C_in * ld, 0.f);
  for (int co = 0; co < C_out; ++co)
    for (int ci = 0; ci < C_in; ++ci)
      for (int kh = 0; kh < KH; ++kh)
        for (int kw = 0; kw < KW; ++kw) {
          float v = w[(((size_t)co * C_in + ci) * KH + kh) * KW + kw];
          if (scale) v = v * scale[co];
          o[((size_t)(kh * KW + kw) * C_in + ci) * ld + co] = v;
        }
  return o;
}

namespace {
__global__ void pack_conv2d_kernel(const float* w, float* out, int C_out, int C_in, int KH, int KW, int ld) {
  const long long n = (long long)KH * KW * C_in * ld;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int co = (int)(i % ld);
  const long long r = i / ld;
  const int ci = (int)(r % C_in);
  const int t = (int)(r / C_in);
  out[i] = co < C_out ? w[(((long long)co * C_in + ci) * KH + t / KW) * KW + t % KW] : 0.f;
}

__global__ void pack_convt2d_phase_kernel(const float* w, float* out, int C_in, int C_out, int KH, int KW, int ld,
                                          ConvT2dTaps t) {
  const long long n = (long long)t.n * C_in * ld;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int co = (int)(i % ld);
  const long long r = i / ld;
  const int ci = (int)(r % C_in);
  const int k = (int)(r / C_in);
  const int kh = t.kh[k], kw = t.kw[k];
  out[i] = (co < C_out && kh >= 0) ? w[(((long long)ci * C_out + co) * KH + kh) * KW + kw] : 0.f;
}

__global__ void insert_zeros_2x_kernel(const float* x, float* out, long long n, int H, int W) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int UW = 2 * W - 1, UH = 2 * H - 1;
  const int u = (int)(i % UW);
  const long long r = i / UW;
  const int v = (int)(r % UH);
  const long long c = r / UH;
  out[i] = ((u | v) & 1) ? 0.f : x[(c * H + (v >> 1)) * W + (u >> 1)];
}

__global__ void avg_pool2_kernel(const float* x, float* out, long long n, int H, int W) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int Wo = W / 2, Ho = H / 2;
  const int j = (int)(i % Wo);
  const long long r = i / Wo;
  const int h = (int)(r % Ho);
  const long long c = r / Ho;
  const float* p = x + (c * H + 2 * h) * W + 2 * j;
  out[i] = ((p[0] + p[1]) + (p[W] + p[W + 1])) * 0.25f;
}
}  // namespace

void launch_pack_conv2d_weight(const float* w, float* out, int C_out, int C_in, int KH, int KW, hipStream_t s) {
  const long long n = (long long)KH * KW * C_in * packed_ld(C_out);
  if (n == 0) return;
  hipLaunchKernelGGL(pack_conv2d_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, w, out, C_out, C_in,
                     KH, KW, packed_ld(C_out));
  check_launch("pack_conv2d");
}

void launch_pack_convt2d_phase(const float* w, float* out, int C_in, int C_out, int KH, int KW, const ConvT2dTaps& t,
                               hipStream_t s) {
  RVC_CHECK(t.n >= 1 && t.n <= kConv2dTapsMax, "pack_convt2d: 1..9 taps");
  const long long n = (long long)t.n * C_in * packed_ld(C_out);
  hipLaunchKernelGGL(pack_convt2d_phase_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, w, out, C_in,
                     C_out, KH, KW, packed_ld(C_out), t);
  check_launch("pack_convt2d_phase");
}

void launch_insert_zeros_2x(const float* x, float* out, long long C, int H, int W, hipStream_t s) {
  const long long n = C * (2LL * H - 1) * (2LL * W - 1);
  if (n <= 0) return;
  hipLaunchKernelGGL(insert_zeros_2x_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, out, n, H, W);
  check_launch("insert_zeros_2x");
}

void launch_avg_pool2(const float* x, float* out, int BC, int H, int W, hipStream_t s) {
  const long long n = (long long)BC * (H / 2) * (W / 2);
  if (n == 0) return;
  hipLaunchKernelGGL(avg_pool2_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, out, n, H, W);
  check_launch("avg_pool2");
}

// ------------------------------------------------------------------ mel front end
// The STFT frames (n_fft 1024, hop 160, reflect padding 512) are read as a
// conv1d over hop-sized blocks: block b holds padded samples [160 b, 160 b +
// 160) as 160 channels, and frame f is taps k = 0..6 over blocks f .. f+6
// (tap 6 uses its first 64 samples).  xb[c][b] = xpad[160 b + c].
namespace {
constexpr int kHop = 160, kPad = 512;

__global__ void rmvpe_blocks_kernel(const float* x, int T, float* xb, int NB) {
  const long long n = (long long)kHop * NB;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int c = (int)(i / NB);
  const int b = (int)(i - (long long)c * NB);
  const long long s = (long long)b * kHop + c;
  float v = 0.f;
  if (s < (long long)T + 2 * kPad) {
    long long p = s - kPad;
    if (p < 0) p = -p;
    else if (p >= T) p = 2LL * (T - 1) - p;
    v = x[p];
  }
  xb[i] = v;
}

__global__ void mel_mag_kernel(const float* S, float* mag, int nbin, int F) {
#pragma clang fp contract(off)
  const long long n = (long long)nbin * F;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float re = S[i];
  const float im = S[i + n];
  mag[i] = sqrtf(re * re + im * im);
}

__global__ void logmel_image_kernel(const float* M, int F, int Fp, int n_mels, float bn_s, float bn_t, float* img,
                                    float* logmel) {
#pragma clang fp contract(off)
  const long long n = (long long)Fp * n_mels;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int f = (int)(i / n_mels);
  const int m = (int)(i - (long long)f * n_mels);
  float v = 0.f;
  if (f < F) {
    v = logf(fmaxf(M[(long long)m * F + f], 1e-5f));
    if (logmel) logmel[(long long)m * F + f] = v;
  }
  img[i] = v * bn_s + bn_t;
}
}  // namespace

void launch_rmvpe_blocks(const float* x, int T, float* xb, int NB, hipStream_t s) {
  const long long n = (long long)kHop * NB;
  hipLaunchKernelGGL(rmvpe_blocks_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, T, xb, NB);
  check_launch("rmvpe_blocks");
}

void launch_mel_mag(const float* S, float* mag, int nbin, int F, hipStream_t s) {
  const long long n = (long long)nbin * F;
  hipLaunchKernelGGL(mel_mag_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, S, mag, nbin, F);
  check_launch("mel_mag");
}

void launch_logmel_image(const float* M, int F, int Fp, int n_mels, float bn_s, float bn_t, float* img,
                         float* logmel, hipStream_t s) {
  const long long n = (long long)Fp * n_mels;
  hipLaunchKernelGGL(logmel_image_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, M, F, Fp, n_mels,
                     bn_s, bn_t, img, logmel);
  check_launch("logmel_image");
}

// ------------------------------------------------------------------ BiGRU
// h_t = GRU(gx_t, h_{t-1}) per direction (PyTorch gate order r, z, n):
//   r = sig(gx_r + W_hr h + b_hr), z = sig(gx_z + W_hz h + b_hz),
//   n = tanh(gx_n + r * (W_hn h + b_hn)),  h = (1 - z) * n + z * h_prev.
// Each direction runs on kGruGroups workgroups of four waves; wave w of group
// g owns units 16 g + 4 w .. +3 and keeps their 12 rows of W_hh in registers
// (lane l: columns 4 l .. 4 l + 3), so the recurrence reads no weights from
// memory.  The waves exchange h through a double buffer of 64-bit words
// (step tag << 32 | float bits), written and read with agent-scope relaxed
// atomics: step s waits until all H words of buffer (s-1)&1 carry tag s-1,
// computes its 4 units and stores them, tagged s, into buffer s&1.  A value
// and its step travel in one single-copy-atomic word, so no fence, counter or
// barrier orders anything; the parity buffers keep a fast wave from
// overwriting a word a slow wave has yet to read (it can only write step s
// after every wave published step s-1, i.e. finished reading step s-2).
// The wait is bounded: past spin_limit polls (or once another wave has given
// up) the wave sets the error flag and returns, so the grid always drains;
// the host reports the flag.
namespace {
constexpr int kGruGroups = 16;
constexpr int kGruUnits = 16;  // per workgroup
constexpr int kGruPollSleep = 1;  // s_sleep units (64 clocks) between two polls

__device__ __forceinline__ unsigned long long gru_word(int tag, float v) {
  return ((unsigned long long)(unsigned)tag << 32) | (unsigned long long)__float_as_uint(v);
}

__global__ void gru_init_kernel(unsigned long long* state, unsigned* sync, int keep_err) {
  // buffer 1 holds h_{-1} = 0 tagged -1; buffer 0 a tag no step waits for
  for (int k = threadIdx.x; k < 2 * 2 * 256; k += blockDim.x) state[k] = gru_word(((k >> 8) & 1) ? -1 : -2, 0.f);
  // sync[2] is the error flag: kept when an earlier GRU's flag still awaits its check
  if (threadIdx.x < 4 && !(threadIdx.x == 2 && keep_err)) sync[threadIdx.x] = 0u;
}

__global__ __launch_bounds__(256) void bigru_kernel(GruArgs g) {
#pragma clang fp contract(off)
  const int d = blockIdx.x / kGruGroups;
  const int gw = blockIdx.x - d * kGruGroups;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int H = g.H;
  const int ub = gw * kGruUnits + wave * 4;
  if (ub >= H) return;  // wave-uniform; no workgroup barrier below
  const float* W = g.whh + (long long)d * 3 * H * H;
  // rows u * 3 + q: unit u's gates r, z, n side by side, so the reduction
  // below leaves unit u's three sums in lanes 16 u .. 16 u + 15
  float wr[12][4];
#pragma unroll
  for (int q = 0; q < 3; ++q)
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int j = ub + u, col = 4 * lane + c;
        wr[u * 3 + q][c] = (j < H && col < H) ? W[(long long)(q * H + j) * H + col] : 0.f;
      }
  const int u = lane >> 4;
  const int ju = ub + u;
  const bool owner = (lane & 15) == 0 && ju < H;
  float bh[3];
#pragma unroll
  for (int q = 0; q < 3; ++q) bh[q] = owner ? g.bhh[(long long)d * 3 * H + q * H + ju] : 0.f;
  unsigned long long* st = g.state + d * 2 * 256;
  unsigned* err = g.sync + 2;

  float hj = 0.f;  // the owner's h_{s-1} (h_{-1} = 0)
  for (int s = 0; s < g.T; ++s) {
    const int t = d == 0 ? s : g.T - 1 - s;
    // gate inputs of this step: issued before the wait
    float gxr = 0.f, gxz = 0.f, gxn = 0.f;
    if (owner) {
      const float* gp = g.gx + d * g.g_d + (long long)t * g.g_t;
      gxr = gp[(long long)ju * g.g_r];
      gxz = gp[(long long)(H + ju) * g.g_r];
      gxn = gp[(long long)(2 * H + ju) * g.g_r];
    }
    // wait for h_{s-1}: all H words of buffer (s-1)&1 tagged s-1.  Every
    // poll issues the lane's four word loads and the error-flag load
    // together (one memory round trip per poll); columns past H read word
    // H - 1, whose tag is awaited like the others (their weights are 0).
    const unsigned long long* hb = st + ((s - 1) & 1) * 256;
    const unsigned want = (unsigned)(s - 1);
    unsigned long long wv[4];
    long long polls = 0;
    for (;;) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        wv[c] = __hip_atomic_load(hb + min(4 * lane + c, H - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const unsigned ev = polls > 0 ? __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
      bool ready = true;
#pragma unroll
      for (int c = 0; c < 4; ++c) ready = ready && (unsigned)(wv[c] >> 32) == want;
      if (__all(ready)) break;
      if (++polls > g.spin_limit || ev != 0u) {
        __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
      }
      __builtin_amdgcn_s_sleep(kGruPollSleep);
    }
    float hv[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) hv[c] = __uint_as_float((unsigned)wv[c]);
    float p[12];
#pragma unroll
    for (int i = 0; i < 12; ++i) p[i] = ((wr[i][0] * hv[0] + wr[i][1] * hv[1]) + wr[i][2] * hv[2]) + wr[i][3] * hv[3];
    // Sums over the 64 lanes, reduce-scatter style, without LDS: a
    // permlane32 swap of rows k and k + 6 leaves lanes 0-31 with row k of
    // lanes l, l + 32 and lanes 32-63 with row k + 6 (the two halves added),
    // a permlane16 swap does the same across 16-lane rows, and DPP mirrors
    // and quad permutations add the last three rows over their 16 lanes.
    // Lane l ends with the rows 3 (l >> 4) .. + 2, the same value in every
    // lane of its 16 (each pair adds the same two terms).
    float a6[6], a3[3];
#pragma unroll
    for (int k = 0; k < 6; ++k) {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(p[k]), __float_as_uint(p[k + 6]), false, false);
      a6[k] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(a6[k]), __float_as_uint(a6[k + 3]), false, false);
      a3[k] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    // row_mirror (l <-> 15 - l), row_half_mirror (l <-> 7 - l), then the
    // quad permutations [2,3,0,1] and [1,0,3,2]
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      a3[k] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a3[k]), 0x140, 0xF, 0xF, false));
      a3[k] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a3[k]), 0x141, 0xF, 0xF, false));
      a3[k] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a3[k]), 0x4E, 0xF, 0xF, false));
      a3[k] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a3[k]), 0xB1, 0xF, 0xF, false));
    }
    if (owner) {
      const float sr = a3[0], sz = a3[1], sn = a3[2];
      const float r = sigmoid_as(gxr + (sr + bh[0]));
      const float zz = sigmoid_as(gxz + (sz + bh[1]));
      const float nn = tanhf(gxn + r * (sn + bh[2]));
      const float h = (1.0f - zz) * nn + zz * hj;
      hj = h;  // h_{s-1} of this unit at the next step: the owner's own word
      __hip_atomic_store(st + (s & 1) * 256 + ju, gru_word(s, h), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      g.out[d * g.o_d + (long long)t * g.o_t + (long long)ju * g.o_j] = h;
    }
  }
}
}  // namespace

void launch_bigru(const GruArgs& g, hipStream_t s) {
  RVC_CHECK(g.T >= 1 && g.H >= 1 && g.H <= kGruGroups * kGruUnits, "bigru: need T >= 1 and 1 <= H <= 256");
  RVC_CHECK(g.state && g.sync && g.gx && g.whh && g.bhh && g.out && g.spin_limit > 0, "bigru: null argument");
  hipLaunchKernelGGL(gru_init_kernel, dim3(1), dim3(256), 0, s, g.state, g.sync, g.keep_err);
  check_launch("gru_init");
  hipLaunchKernelGGL(bigru_kernel, dim3(2 * kGruGroups), dim3(256), 0, s, g);
  check_launch("bigru");
}

// ------------------------------------------------------------------ decode
// One wave per frame: argmax over the nb bins (first maximum on ties), then
// the salience-weighted mean of the cents of bins c-4 .. c+4 (zero outside;
// both 9-term sums in numpy's pairwise order), 0 when the frame's maximum
// (with the zero padding) is <= thred, f0 = 10 * 2^(cents / 1200) with
// exactly 10 Hz mapped to 0 (runtime/models/rmvpe.py:899-924).
namespace {
__global__ __launch_bounds__(256) void rmvpe_decode_kernel(const float* sal, long long s_f, long long s_k, int F,
                                                           int nb, const float* cents, float thred, float* f0) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int f = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (f >= F) return;
  const float* row = sal + (long long)f * s_f;
  float best = -INFINITY;
  int bi = 0;
  for (int k = lane; k < nb; k += 64) {
    const float v = row[(long long)k * s_k];
    if (v > best) {
      best = v;
      bi = k;
    }
  }
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(best, off);
    const int oi = __shfl_xor(bi, off);
    if (ov > best || (ov == best && oi < bi)) {
      best = ov;
      bi = oi;
    }
  }
  if (lane != 0) return;
  float pv[9], sv[9];
#pragma unroll
  for (int i = 0; i < 9; ++i) {
    const int k = bi - 4 + i;
    const float sk = (k >= 0 && k < nb) ? row[(long long)k * s_k] : 0.f;
    sv[i] = sk;
    pv[i] = sk * cents[bi + i];
  }
  const float ps = (((pv[0] + pv[1]) + (pv[2] + pv[3])) + ((pv[4] + pv[5]) + (pv[6] + pv[7]))) + pv[8];
  const float ws = (((sv[0] + sv[1]) + (sv[2] + sv[3])) + ((sv[4] + sv[5]) + (sv[6] + sv[7]))) + sv[8];
  float c = ps / ws;
  const float mx = fmaxf(best, 0.f);
  if (mx <= thred) c = 0.f;
  float y = 10.0f * powf(2.0f, c / 1200.0f);
  if (y == 10.0f) y = 0.f;
  f0[f] = y;
}
}  // namespace

void launch_rmvpe_decode(const float* sal, long long s_f, long long s_k, int F, int nb, const float* cents,
                         float thred, float* f0, hipStream_t s) {
  RVC_CHECK(nb >= 1 && F >= 0, "rmvpe_decode: invalid shape");
  if (F == 0) return;
  hipLaunchKernelGGL(rmvpe_decode_kernel, dim3((unsigned)((F + 3) / 4)), dim3(256), 0, s, sal, s_f, s_k, F, nb,
                     cents, thred, f0);
  check_launch("rmvpe_decode");
}

}  // namespace rvc
