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
//
// The bf16 form (BF = true, config 5) runs the same tiles and epilogue on
// v_mfma_f32_16x16x32_bf16 with 32-channel chunks: lane l supplies the eight
// channels c + 8*(l/16) .. +7 of row co_tile + l%16 (A) and of column
// m_tile + l%16 + 1 - j (B) -- only the pairing of A's and B's channel slots
// matters -- so LDS holds both operands channel-contiguous, xs[m][ci] and
// ws[k][co][ci] with row stride 40 bf16 (80 bytes: the 16 rows of one read
// fall on 16 distinct groups of four banks), and each fragment is one 16-byte
// read.  The input is rounded to bf16 (nearest even) after the leaky ReLU as
// it is staged, two channels per 32-bit LDS word; the weights arrive packed
// in bf16.  Products of two bf16 values are exact in fp32, the sums are fp32.
#include <algorithm>

#include "internal.h"

namespace rvc {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

namespace {

// two floats -> two bf16 (round to nearest even) in one 32-bit word, lo first
__device__ __forceinline__ uint32_t ct_pack_bf16x2(float lo, float hi) {
  uint32_t a = __float_as_uint(lo), b = __float_as_uint(hi);
  a += 0x7fffu + ((a >> 16) & 1u);
  b += 0x7fffu + ((b >> 16) & 1u);
  return (a >> 16) | (b & 0xffff0000u);
}

// The bf16 staging layout of one chunk of BK channels (BK = 32)
template <int K, int BM, int BN, int NT, int BK>
struct CtB16 {
  static constexpr int RS = BK + 8;                   // LDS row stride (bf16)
  static constexpr int XW = BN + 1;                   // window m0-1 .. m0+BN-1
  static constexpr int XP = (BK / 2) * XW;            // channel pairs of the window
  static constexpr int WV = K * BM * (BK / 8);        // 16-byte weight vectors
  static constexpr int XPT = (XP + NT - 1) / NT;
  static constexpr int WPT = (WV + NT - 1) / NT;
  static constexpr int XH = XW * RS;                  // bf16 elements of xs
  static constexpr int STAGE = XH + K * BM * RS;      // bf16 elements per stage (XH*2 bytes is a multiple of 16)
};

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

template <int K, int S, int TM, int TN, int WMW, int WNW, int BK, bool FUSED, bool BF>
// (the bf16 staging holds channel pairs of a 32-channel chunk: one resident wave less)
__global__ __launch_bounds__(64 * WMW * WNW)
__attribute__((amdgpu_waves_per_eu(ct_waves_per_eu<K, S, TM, TN>() - (BF && ct_waves_per_eu<K, S, TM, TN>() > 3 ? 1 : 0))))
void convt_os_kernel(ConvTOsLaunch a) {
  using C = CtCfg<K, S, TM, TN, WMW, WNW, BK>;
  constexpr int BM = C::BM, BN = C::BN, NT = C::NT, XW = C::XW, XPT = C::XPT, WPT = C::WPT;
  extern __shared__ __attribute__((aligned(16))) float smem[];

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

  floatx4 acc[S][TM][TN];
#pragma unroll
  for (int r = 0; r < S; ++r)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int n = 0; n < TN; ++n) acc[r][i][n] = floatx4{0.f, 0.f, 0.f, 0.f};
  if constexpr (BF) {
    using D = CtB16<K, BM, BN, NT, BK>;
    constexpr int RS = D::RS;
    constexpr unsigned kOut = 0x80000000u;
    uint16_t* sm16 = reinterpret_cast<uint16_t*>(smem);
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.x + (long long)b * a.xb), (short)0, (int)(4u * (unsigned)(a.C_in * a.L_in)), 0x00020000);
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.w16, (short)0, (int)(2u * (unsigned)(a.K * a.C_out * a.w16_ld)), 0x00020000);
    // pair p = cp * XW + mpos: channels 2cp, 2cp+1 of window column mpos
    unsigned xo[D::XPT], wo[D::WPT];
#pragma unroll
    for (int e = 0; e < D::XPT; ++e) {
      const int p = tid + e * NT;
      const int cp = p / XW, mpos = p - cp * XW;
      const int mi = m0 - 1 + mpos;
      xo[e] = p < D::XP && mi >= 0 && mi < a.L_in ? 4u * (unsigned)(2 * cp * a.L_in + mi) : kOut;
    }
    // vector v = row * (BK / 8) + part, row = k * BM + co
#pragma unroll
    for (int e = 0; e < D::WPT; ++e) {
      const int v = tid + e * NT;
      const int row = v / (BK / 8), part = v - row * (BK / 8);
      const int k = row / BM, co = row - k * BM;
      wo[e] = v < D::WV ? 2u * (unsigned)((k * a.C_out + co0 + co) * a.w16_ld + 8 * part) : kOut;
    }
    float x0[D::XPT], x1[D::XPT];
    uint4 wv[D::WPT];
    auto gload = [&](int ci0) {
      const unsigned xadd = 4u * (unsigned)(ci0 * a.L_in), wadd = 2u * (unsigned)ci0;
      const unsigned row1 = 4u * (unsigned)a.L_in;
#pragma unroll
      for (int e = 0; e < D::XPT; ++e) {
        const unsigned o = xo[e] == kOut ? kOut : xo[e] + xadd;
        x0[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xrs, o, 0, 0));
        x1[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xrs, o == kOut ? kOut : o + row1, 0, 0));
      }
#pragma unroll
      for (int e = 0; e < D::WPT; ++e)
        wv[e] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wrs, wo[e] == kOut ? kOut : wo[e] + wadd, 0, 0));
    };
    auto lstore = [&](int buf) {
      uint16_t* xs = sm16 + buf * D::STAGE;
      uint16_t* ws = xs + D::XH;
#pragma unroll
      for (int e = 0; e < D::XPT; ++e) {
        const int p = tid + e * NT;
        if (p < D::XP) {
          const int cp = p / XW, mpos = p - cp * XW;
          float u = x0[e], v = x1[e];
          u = u >= 0.f ? u : u * a.in_slope;
          v = v >= 0.f ? v : v * a.in_slope;
          *reinterpret_cast<uint32_t*>(xs + mpos * RS + 2 * cp) = ct_pack_bf16x2(u, v);
        }
      }
#pragma unroll
      for (int e = 0; e < D::WPT; ++e) {
        const int v = tid + e * NT;
        if (v < D::WV) {
          const int row = v / (BK / 8), part = v - row * (BK / 8);
          *reinterpret_cast<uint4*>(ws + row * RS + 8 * part) = wv[e];
        }
      }
    };
    const int nchunk = a.C_in / BK;  // the launcher requires C_in % BK == 0
    gload(0);
    lstore(0);
    __syncthreads();
    int buf = 0;
    for (int c = 0; c < nchunk; ++c) {
      if (c + 1 < nchunk) gload((c + 1) * BK);
      const uint16_t* xs = sm16 + buf * D::STAGE;
      const uint16_t* ws = xs + D::XH;
      const uint16_t* xl = xs + (wn * TN * 16 + l16) * RS + 8 * kq;
      const uint16_t* wl = ws + (wm * TM * 16 + l16) * RS + 8 * kq;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        bf16x8 bv[TN];
#pragma unroll
        for (int n = 0; n < TN; ++n) {
          uint4 t = *reinterpret_cast<const uint4*>(xl + (n * 16 + 1 - j) * RS);
          __builtin_memcpy(&bv[n], &t, 16);
        }
#pragma unroll
        for (int r = 0; r < S; ++r) {
          const int k = r + j * S;
          if (k < K) {
            bf16x8 av[TM];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
              uint4 t = *reinterpret_cast<const uint4*>(wl + (k * BM + i * 16) * RS);
              __builtin_memcpy(&av[i], &t, 16);
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
              for (int n = 0; n < TN; ++n)
                acc[r][i][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i], bv[n], acc[r][i][n], 0, 0, 0);
          }
        }
      }
      if (c + 1 < nchunk) lstore(buf ^ 1);
      __syncthreads();
      buf ^= 1;
    }
  } else {
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
      const unsigned off = e < nh && hi >= 0 && hi < a.N ? 4u * (unsigned)hi : kBufOut;
      hs[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(hrs, off, 0, 0));
    }
    for (int e = tid; e < BM * kNoiseTapsMax; e += NT) {
      const int row = e / kNoiseTapsMax, t = e - row * kNoiseTapsMax;
      nws[e] = t < a.kn ? a.nw[(co0 + row) * a.kn + t] : 0.f;
    }
    __syncthreads();
  }
  // The tile's outputs [BM rows][BN * S columns]: a lane's values of one row
  // are S apart in memory (one per phase), so stored straight from the
  // accumulators every cache line is written in S pieces.  kStageOut: they
  // go out through LDS instead, staged as rows, consecutive lanes storing
  // consecutive floats (bf16 upsamplers 0.64 -> 0.52 ms at B = 4; the fp32
  // stride-10 tiles 3 % faster, the fp32 stride-2 tiles 6 % slower, so
  // those keep the direct stores).
  constexpr bool kStageOut = BF || S > 2;
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
          if constexpr (kStageOut)
            acc[r][i][n][g] = v;
          else if (ok)
            ob[oi] = v;
        }
      }
    }
  }
  if constexpr (kStageOut) {
    constexpr int OTW = BN * S + 1;  // row stride (floats) of the staged tile
    float* ot = smem;
    __syncthreads();  // every wave has read the noise window and weights
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int lrow = wm * TM * 16 + i * 16 + 4 * kq;
#pragma unroll
      for (int n = 0; n < TN; ++n) {
        const int ml = wn * TN * 16 + n * 16 + l16;
#pragma unroll
        for (int r = 0; r < S; ++r)
#pragma unroll
          for (int g = 0; g < 4; ++g) ot[(lrow + g) * OTW + ml * S + r] = acc[r][i][n][g];
      }
    }
    __syncthreads();
    const int o0 = m0 * S - a.pad;
    const int ncol = min(BN * S, a.L_out - o0);  // columns of this tile inside [.., L_out)
    for (int e = tid; e < BM * BN * S; e += NT) {
      const int row = e / (BN * S), col = e - row * (BN * S);
      const int o = o0 + col;
      if (col < ncol && o >= 0) ob[(long long)(co0 + row) * a.oc + o] = ot[row * OTW + col];
    }
  }
}

template <int K, int S, int TM, int TN, int WMW, int WNW, int BK, bool FUSED, bool BF>
bool launch_one(const ConvTOsLaunch& a, hipStream_t s) {
  using C = CtCfg<K, S, TM, TN, WMW, WNW, BK>;
  if (a.C_out % C::BM != 0 || a.C_in % BK != 0) return false;
  const int nh = C::BN * S * a.ns + a.kn - a.ns;
  const size_t epi = (size_t)(nh + kNoiseTapsMax + 3) / 4 * 4 + (size_t)C::BM * kNoiseTapsMax;
  const size_t stage = BF ? 2 * (size_t)CtB16<K, C::BM, C::BN, C::NT, BK>::STAGE : sizeof(float) * C::STAGE;
  const size_t otile = BF || S > 2 ? sizeof(float) * C::BM * (C::BN * S + 1) : 0;  // the staged output tile
  const size_t lds = std::max<size_t>(std::max<size_t>(2 * stage, otile), a.noise ? 0 : sizeof(float) * epi);
  constexpr int kMax = BF ? 96 * 1024 : 65536;  // bf16: the 24-tap stage needs 72 KB
  if (lds > (size_t)kMax) return false;
  static bool attr = false;
  if (!attr) {
    RVC_HIP(hipFuncSetAttribute((const void*)convt_os_kernel<K, S, TM, TN, WMW, WNW, BK, FUSED, BF>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, kMax));
    attr = true;
  }
  const long long grid = (long long)a.B * (a.C_out / C::BM) * ((a.M + C::BN - 1) / C::BN);
  RVC_CHECK(grid < (1LL << 31), "convt_os: launch too large");
  launch_timed(convt_os_kernel<K, S, TM, TN, WMW, WNW, BK, FUSED, BF>, dim3((unsigned)grid), dim3(C::NT), lds, s, a);
  check_launch("convt_os");
  return true;
}

template <int K, int S, int TM, int TN, int WMW, int WNW, int BK, bool BF = false>
bool launch_cfg(const ConvTOsLaunch& a, hipStream_t s) {
  return a.noise ? launch_one<K, S, TM, TN, WMW, WNW, BK, false, BF>(a, s)
                 : launch_one<K, S, TM, TN, WMW, WNW, BK, true, BF>(a, s);
}

}  // namespace

bool convt_os_supported(int K, int S) {
  return (K == 16 && S == 10) || (K == 20 && S == 10) || (K == 24 && S == 12) || (K == 4 && S == 2);
}

bool launch_convt_os(const ConvTOsLaunch& a, hipStream_t s) {
  RVC_CHECK(a.x && (a.w || a.w16) && a.out && a.B >= 1 && a.C_in >= 1 && a.C_out >= 1 && a.L_in >= 1 && a.L_out >= 1,
            "convt_os: invalid launch");
  if (a.w16) {
    RVC_CHECK(a.w16_ld % 8 == 0 && a.w16_ld >= a.C_in && (reinterpret_cast<uintptr_t>(a.w16) & 15) == 0 &&
                  2LL * a.K * a.C_out * a.w16_ld < (1LL << 31),
              "convt_os: bf16 weights must be 16-byte rows of at least C_in");
  } else {
    RVC_CHECK(a.w_ld % 4 == 0 && (reinterpret_cast<uintptr_t>(a.w) & 15) == 0,
              "convt_os: weights must be 16-byte rows");
  }
  RVC_CHECK(a.noise || (a.har && a.nw && a.kn >= 1 && a.kn <= kNoiseTapsMax && a.ns >= 1),
            "convt_os: the noise term needs a tensor or har + weights with <= 8 taps");
  RVC_CHECK(a.M == (a.L_out + a.pad + a.S - 1) / a.S, "convt_os: M must cover every output");
  RVC_CHECK((long long)a.C_out * a.oc < (1LL << 31) && 4LL * a.C_in * a.L_in < (1LL << 31) &&
                (a.w16 || 4LL * a.K * a.C_in * a.w_ld < (1LL << 31)),
            "convt_os: per-batch-item tensors must stay below 2^31 bytes (32-bit buffer offsets)");
  // Long strides (S = 10, 12): one wave holds S accumulator sets of one
  // 16 x 16 tile; 16 x 64 tiles of 4 waves, three per CU (LDS), so the last
  // partial round of a launch is short.  Stride 2: 32 x 128 tiles of 2 x 2
  // waves, each a 16 x 64 strip.
  if (a.w16) {
    // the same tiles on 32-channel bf16 chunks
    if (a.K == 16 && a.S == 10) return launch_cfg<16, 10, 1, 1, 1, 4, 32, true>(a, s);
    if (a.K == 20 && a.S == 10) return launch_cfg<20, 10, 1, 1, 1, 4, 32, true>(a, s);
    if (a.K == 24 && a.S == 12) return launch_cfg<24, 12, 1, 1, 1, 4, 32, true>(a, s);
    if (a.K == 4 && a.S == 2) return launch_cfg<4, 2, 1, 4, 2, 2, 32, true>(a, s);
    return false;
  }
  if (a.K == 16 && a.S == 10) return launch_cfg<16, 10, 1, 1, 1, 4, 16>(a, s);
  if (a.K == 20 && a.S == 10) return launch_cfg<20, 10, 1, 1, 1, 4, 16>(a, s);
  if (a.K == 24 && a.S == 12) return launch_cfg<24, 12, 1, 1, 1, 4, 8>(a, s);  // 16-channel chunks exceed 64 KB
  if (a.K == 4 && a.S == 2) return launch_cfg<4, 2, 1, 4, 2, 2, 16>(a, s);
  return false;
}

}  // namespace rvc
