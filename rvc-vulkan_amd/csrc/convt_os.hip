// Output-stationary polyphase ConvTranspose1d for the GeneratorNSF upsample
// stack, with the stage's NSF noise term and the bias in the epilogue, on
// fp32 matrix cores (v_mfma_f32_16x16x4_f32).
//
//   out[b][co][o] = (sum_{ci,k} W[ci][co][k] * lrelu(x[b][ci][m - j]) + bias[co]) + noise[b][co][o]
//   with o + pad = m*S + r (0 <= r < S) and k = r + j*S,
//
// i.e. ups_i(lrelu(x)) + noise_conv_i(har) of runtime/models/vits.py:2196-2210
// (runtime/nn.py:293-346 for the transposed convolution).  The noise term is
// either a precomputed tensor [B][C_out][L_out] or, for short noise kernels,
// the one-channel strided convolution of the harmonic source computed here:
//   noise[b][co][o] = (sum_{t<kn} nw[co][t] * har[b][o*ns - np + t]) + nb[co].
//
// A workgroup owns BM output channels x BN input positions m and so the BN*S
// contiguous outputs o = m*S + r - pad of every phase r.  Per chunk of BK
// input channels it stages the input window x[ci][m0-1 .. m0+BN) once (every
// phase and shift reads it) and the packed weights of all K taps.  For each
// shift j the B operand (x shifted by j) is read once and multiplied with
// the A operands of every phase r whose tap r + j*S exists, so a wave holds
// S accumulator sets -- all phases of its outputs -- and nothing is written
// before the epilogue.  There each output is formed once: acc + bias, plus
// the noise term, and stored.  Compared with one grid per phase (each phase
// storing every S-th sample and accumulating onto a noise buffer), every
// output line is written once and the noise tensor is neither written nor
// re-read for the stages that compute it here.
//
// Lane l of an MFMA step supplies A = W[k][c + l/16][co_tile + l%16] and
// B = xs[c + l/16][m_tile + l%16 + 1 - j]; its accumulator i holds row
// co_tile + 4*(l/16) + i, column m_tile + l%16.
#include <algorithm>

#include "internal.h"

namespace rvc {

typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

// K taps of stride S (K <= 2S: at most two shifts j per phase); waves are
// WMW x WNW, each owning TM x TN tiles of 16 x 16.
template <int K, int S, int TM, int TN, int WMW, int WNW, int BK>
struct CtCfg {
  static_assert(K <= 2 * S && K > S, "two shifts per phase");
  static_assert(BK % 4 == 0, "channel chunk of whole MFMA steps");
  static constexpr int BM = WMW * TM * 16;
  static constexpr int BN = WNW * TN * 16;
  static constexpr int NT = 64 * WMW * WNW;
  static constexpr int XW = BN + 1;  // window m0-1 .. m0+BN-1
  static constexpr int XN = BK * XW;
  static constexpr int WN4 = K * BK * BM / 4;
  static constexpr int XPT = (XN + NT - 1) / NT;
  static constexpr int WPT = (WN4 + NT - 1) / NT;
  static constexpr int STAGE = (XN + 4 * WN4 + 3) / 4 * 4;
};

// FUSED: the noise conv is computed here from har (else read from a.noise)
// Resident waves per SIMD the register budget is held to: S accumulator sets
// of TM x TN tiles take 4*S*TM*TN registers, and the A operands of up to K
// taps are read ahead.
template <int K, int S, int TM, int TN>
constexpr int ct_waves_per_eu() {
  return (4 * S * TM * TN > 40 || K > 16) ? 3 : (4 * S * TM * TN > 32 ? 4 : 5);
}

template <int K, int S, int TM, int TN, int WMW, int WNW, int BK, bool FUSED>
__global__ __launch_bounds__(64 * WMW * WNW) __attribute__((amdgpu_waves_per_eu(ct_waves_per_eu<K, S, TM, TN>())))
void convt_os_kernel(ConvTOsLaunch a) {
  using C = CtCfg<K, S, TM, TN, WMW, WNW, BK>;
  constexpr int BM = C::BM, BN = C::BN, NT = C::NT, XW = C::XW, XPT = C::XPT, WPT = C::WPT;
  extern __shared__ float smem[];

  const int n_co = a.C_out / BM;
  const int n_m = (a.M + BN - 1) / BN;
  // tile order: the C_out tiles of one m tile read the same input window;
  // they are dealt 8 dispatch slots apart, onto one XCD (and its L2)
  const int per_b = n_co * n_m;
  const int b = blockIdx.x / per_b;
  const int lin = blockIdx.x - b * per_b;
  int tm, tco;
  if (n_co > 1) {
    const int full = (n_m / 8) * 8 * n_co;
    if (lin < full) {
      tm = (lin / (8 * n_co)) * 8 + lin % 8;
      tco = (lin / 8) % n_co;
    } else {
      tm = (n_m / 8) * 8 + (lin - full) / n_co;
      tco = (lin - full) % n_co;
    }
  } else {
    tm = lin;
    tco = 0;
  }
  const int m0 = tm * BN;
  const int co0 = tco * BM;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WMW;
  const int wn = wave / WMW;
  const int kq = lane >> 4;
  const int l16 = lane & 15;

  // Staging loads go through buffer resources over this batch item's input
  // and the packed weights (32-bit offsets; an out-of-range offset reads 0,
  // which is the zero padding outside [0, L_in)).
  constexpr unsigned kOut = 0x80000000u;
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.x + (long long)b * a.xb), (short)0, (int)(4u * (unsigned)(a.C_in * a.L_in)), 0x00020000);
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.w, (short)0, (int)(4u * (unsigned)(a.K * a.C_in * a.w_ld)), 0x00020000);
  // staging offsets of chunk 0 (bytes); chunk c adds c*BK rows
  unsigned xo[XPT], wo[WPT];
#pragma unroll
  for (int e = 0; e < XPT; ++e) {
    const int idx = tid + e * NT;
    const int row = idx / XW;
    const int mi = m0 - 1 + idx - row * XW;
    xo[e] = idx < C::XN && mi >= 0 && mi < a.L_in ? 4u * (unsigned)(row * a.L_in + mi) : kOut;
  }
#pragma unroll
  for (int e = 0; e < WPT; ++e) {
    const int idx = tid + e * NT;
    const int row = idx / (BM / 4);  // (tap, channel) row of the chunk
    const int c4 = idx - row * (BM / 4);
    const int k = row / BK;
    wo[e] = idx < C::WN4 ? 4u * (unsigned)((k * a.C_in + row - k * BK) * a.w_ld + co0 + 4 * c4) : kOut;
  }
  float xv[XPT];
  float4 wreg[WPT];
  auto gload = [&](int ci0) {
    const unsigned xadd = 4u * (unsigned)(ci0 * a.L_in), wadd = 4u * (unsigned)(ci0 * a.w_ld);
#pragma unroll
    for (int e = 0; e < XPT; ++e)
      xv[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xrs, xo[e] == kOut ? kOut : xo[e] + xadd, 0, 0));
#pragma unroll
    for (int e = 0; e < WPT; ++e)
      wreg[e] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(wrs, wo[e] == kOut ? kOut : wo[e] + wadd, 0, 0));
  };
  auto lstore = [&](int buf) {
    float* xs = smem + buf * C::STAGE;
    float* ws = xs + C::XN;
#pragma unroll
    for (int e = 0; e < XPT; ++e) {
      const int idx = tid + e * NT;
      if (idx < C::XN) {
        const float v = xv[e];
        xs[idx] = v >= 0.f ? v : v * a.in_slope;
      }
    }
#pragma unroll
    for (int e = 0; e < WPT; ++e) {
      const int idx = tid + e * NT;
      if (idx < C::WN4) reinterpret_cast<float4*>(ws)[idx] = wreg[e];
    }
  };

  floatx4 acc[S][TM][TN];
#pragma unroll
  for (int r = 0; r < S; ++r)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int n = 0; n < TN; ++n) acc[r][i][n] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int nchunk = a.C_in / BK;  // the launcher requires C_in % BK == 0
  gload(0);
  lstore(0);
  __syncthreads();
  int buf = 0;
  for (int c = 0; c < nchunk; ++c) {
    if (c + 1 < nchunk) gload((c + 1) * BK);
    const float* xs = smem + buf * C::STAGE;
    const float* ws = xs + C::XN;
    const float* xl = xs + kq * XW + wn * TN * 16 + l16;
    const float* wl = ws + kq * BM + wm * TM * 16 + l16;
#pragma unroll
    for (int q = 0; q < BK / 4; ++q) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        float bv[TN];
#pragma unroll
        for (int n = 0; n < TN; ++n) bv[n] = xl[4 * q * XW + n * 16 + 1 - j];
#pragma unroll
        for (int r = 0; r < S; ++r) {
          const int k = r + j * S;
          if (k < K) {
            float av[TM];
#pragma unroll
            for (int i = 0; i < TM; ++i) av[i] = wl[(k * BK + 4 * q) * BM + i * 16];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
              for (int n = 0; n < TN; ++n)
                acc[r][i][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[n], acc[r][i][n], 0, 0, 0);
          }
        }
      }
    }
    if (c + 1 < nchunk) lstore(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }

  // ---- epilogue: out = (acc + bias) + noise ----
  // The noise conv's input window of this tile's outputs
  // o in [m0*S - pad, (m0+BN)*S - pad): har[o*ns - np + t], t < kn, and the
  // tile's noise weights go to LDS (the staging buffers are dead: every wave
  // passed the last barrier), both zero-padded to kNoiseTapsMax taps so every
  // output takes the same branch-free kNoiseTapsMax-term sum; the padded
  // terms are exact zeros after the kn real ones.
  const long long hlo = (long long)(m0 * S - a.pad) * a.ns - a.np;
  const int nh = BN * S * a.ns + a.kn - a.ns;
  const int nhp = (nh + kNoiseTapsMax + 3) / 4 * 4;
  float* hs = smem;
  float* nws = smem + nhp;  // [BM][kNoiseTapsMax]
  constexpr bool fused = FUSED;
  if (fused) {
    const __amdgpu_buffer_rsrc_t hrs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.har + (long long)b * a.harb), (short)0, (int)(4u * (unsigned)a.N), 0x00020000);
    for (int e = tid; e < nhp; e += NT) {
      const long long hi = hlo + e;
      const unsigned off = e < nh && hi >= 0 && hi < a.N ? 4u * (unsigned)hi : kOut;
      hs[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(hrs, off, 0, 0));
    }
    for (int e = tid; e < BM * kNoiseTapsMax; e += NT) {
      const int row = e / kNoiseTapsMax, t = e - row * kNoiseTapsMax;
      nws[e] = t < a.kn ? a.nw[(co0 + row) * a.kn + t] : 0.f;
    }
    __syncthreads();
  }
  float* ob = a.out + (long long)b * a.ob;
  const float* nbt = fused ? nullptr : a.noise + (long long)b * a.ob;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int lrow = wm * TM * 16 + i * 16 + 4 * kq;  // rows co0 + lrow .. + 3
    const int cb = co0 + lrow;
    float bias[4], nbias[4], nwr[4][kNoiseTapsMax];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      bias[g] = a.bias ? a.bias[cb + g] : 0.f;
      nbias[g] = fused && a.nb ? a.nb[cb + g] : 0.f;
#pragma unroll
      for (int t = 0; t < kNoiseTapsMax; ++t) nwr[g][t] = fused ? nws[(lrow + g) * kNoiseTapsMax + t] : 0.f;
    }
#pragma unroll
    for (int n = 0; n < TN; ++n) {
      const int ml = wn * TN * 16 + n * 16 + l16;  // column within the tile
      const int m = m0 + ml;
#pragma unroll
      for (int r = 0; r < S; ++r) {
        const int o = m * S + r - a.pad;
        const bool ok = o >= 0 && o < a.L_out;
        float h[kNoiseTapsMax];
        const int hoff = (ml * S + r) * a.ns;
#pragma unroll
        for (int t = 0; t < kNoiseTapsMax; ++t) h[t] = fused ? hs[hoff + t] : 0.f;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const long long oi = (long long)(cb + g) * a.oc + o;
          float nv;
          if (fused) {
            float sum = nwr[g][0] * h[0];
#pragma unroll
            for (int t = 1; t < kNoiseTapsMax; ++t) sum = sum + nwr[g][t] * h[t];
            nv = sum + nbias[g];
          } else {
            nv = ok ? nbt[oi] : 0.f;
          }
          const float v = (acc[r][i][n][g] + bias[g]) + nv;
          if (ok) ob[oi] = v;
        }
      }
    }
  }
}

template <int K, int S, int TM, int TN, int WMW, int WNW, int BK, bool FUSED>
bool launch_one(const ConvTOsLaunch& a, hipStream_t s) {
  using C = CtCfg<K, S, TM, TN, WMW, WNW, BK>;
  if (a.C_out % C::BM != 0 || a.C_in % BK != 0) return false;
  const int nh = C::BN * S * a.ns + a.kn - a.ns;
  const size_t epi = (size_t)(nh + kNoiseTapsMax + 3) / 4 * 4 + (size_t)C::BM * kNoiseTapsMax;
  const size_t lds = sizeof(float) * std::max<size_t>(2 * C::STAGE, a.noise ? 0 : epi);
  if (lds > 65536) return false;
  static bool attr = false;
  if (!attr) {
    RVC_HIP(hipFuncSetAttribute((const void*)convt_os_kernel<K, S, TM, TN, WMW, WNW, BK, FUSED>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 65536));
    attr = true;
  }
  const long long grid = (long long)a.B * (a.C_out / C::BM) * ((a.M + C::BN - 1) / C::BN);
  RVC_CHECK(grid < (1LL << 31), "convt_os: launch too large");
  hipLaunchKernelGGL((convt_os_kernel<K, S, TM, TN, WMW, WNW, BK, FUSED>), dim3((unsigned)grid), dim3(C::NT), lds, s,
                     a);
  check_launch("convt_os");
  return true;
}

template <int K, int S, int TM, int TN, int WMW, int WNW, int BK>
bool launch_cfg(const ConvTOsLaunch& a, hipStream_t s) {
  return a.noise ? launch_one<K, S, TM, TN, WMW, WNW, BK, false>(a, s) : launch_one<K, S, TM, TN, WMW, WNW, BK, true>(a, s);
}

}  // namespace

bool convt_os_supported(int K, int S) {
  return (K == 16 && S == 10) || (K == 20 && S == 10) || (K == 24 && S == 12) || (K == 4 && S == 2);
}

bool launch_convt_os(const ConvTOsLaunch& a, hipStream_t s) {
  RVC_CHECK(a.x && a.w && a.out && a.B >= 1 && a.C_in >= 1 && a.C_out >= 1 && a.L_in >= 1 && a.L_out >= 1,
            "convt_os: invalid launch");
  RVC_CHECK(a.w_ld % 4 == 0 && (reinterpret_cast<uintptr_t>(a.w) & 15) == 0, "convt_os: weights must be 16-byte rows");
  RVC_CHECK(a.noise || (a.har && a.nw && a.kn >= 1 && a.kn <= kNoiseTapsMax && a.ns >= 1),
            "convt_os: the noise term needs a tensor or har + weights with <= 8 taps");
  RVC_CHECK(a.M == (a.L_out + a.pad + a.S - 1) / a.S, "convt_os: M must cover every output");
  RVC_CHECK((long long)a.C_out * a.oc < (1LL << 31) && 4LL * a.C_in * a.L_in < (1LL << 31) &&
                4LL * a.K * a.C_in * a.w_ld < (1LL << 31),
            "convt_os: per-batch-item tensors must stay below 2^31 bytes (32-bit buffer offsets)");
  // Long strides (S = 10, 12): one wave holds S accumulator sets of one
  // 16 x 16 tile; 16 x 64 tiles of 4 waves, three per CU (LDS), so the last
  // partial round of a launch is short.  Stride 2: 32 x 128 tiles of 2 x 2
  // waves, each a 16 x 64 strip.
  if (a.K == 16 && a.S == 10) return launch_cfg<16, 10, 1, 1, 1, 4, 16>(a, s);
  if (a.K == 20 && a.S == 10) return launch_cfg<20, 10, 1, 1, 1, 4, 16>(a, s);
  if (a.K == 24 && a.S == 12) return launch_cfg<24, 12, 1, 1, 1, 4, 8>(a, s);  // 16-channel chunks exceed 64 KB
  if (a.K == 4 && a.S == 2) return launch_cfg<4, 2, 1, 4, 2, 2, 16>(a, s);
  return false;
}

}  // namespace rvc
