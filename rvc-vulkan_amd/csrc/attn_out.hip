// enc_p's attention output block as one kernel (runtime/models/vits.py:
// 1018-1049, the attention layer's conv_o, the residual and norm_layers_1):
//
//   a[c][t]   = the attention output: the key-split partials merged
//               (m, l, O per slice; out = sum_s O_s e^(m_s - M) /
//               sum_s l_s e^(m_s - M), M = max_s m_s), or the merged
//               tensor itself
//   y[co][t]  = (sum_ci W_o[co][ci] a[ci][t] + b_o[co]) + x[co][t]
//   out[co][t]= (y - mean_t) / sqrt(var_t + eps) * g[co] + beta[co]
//
// with mean / var over the C channels of frame t (two-pass, float64 sums, the
// formulas of layernorm_cols_wave_kernel).  It replaces three launches (the
// merge, conv_o, the LayerNorm): the LayerNorm needs every channel of a frame,
// and so does the merge's consumer, so a workgroup owns BN = 16 frames and all
// C = 16 * RT channels.  Wave w computes output rows [16w, 16w + 16) over the
// whole reduction with v_mfma_f32_16x16x4_f32: its weights go straight from
// global memory into registers (each weight is read once per workgroup), the
// merged attention tile a[C][16] sits in LDS as the B operand.  Weight,
// bias, residual and the first partial-sum loads are all issued before the
// merge's first barrier.
#include "internal.h"

namespace rvc {

typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int BN = 16;         // frames per workgroup
constexpr int kMaxKS = 8;      // key splits a launch merges (all loads in flight together)

// KSM = 1: the attention output is already merged (a.att); KSM = kMaxKS:
// a.KS <= KSM partial slices in a.part.  Every global access is a buffer
// load at a 32-bit offset (the launcher bounds the tensors), masked lanes
// pass kBufOut and read 0.
template <int RT, int KSM>
__global__ __launch_bounds__(64 * RT) void attn_out_ln_kernel(AttnOutArgs a) {
  constexpr int C = 16 * RT;
  constexpr int NT = 64 * RT;
  constexpr int EPT = C * BN / NT;  // merged elements per thread (4)
  __shared__ float xs[C * BN];      // a[ci][col], then y[co][col]
  __shared__ double red[NT / BN][BN];
  __shared__ float stat[2][BN];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int kq = lane >> 4;
  const int l16 = lane & 15;
  const int b = blockIdx.y;
  const int t0 = blockIdx.x * BN;
  const int P = a.P, D = a.D, H = a.H, KS = a.KS;
  const int col = tid % BN;  // the column this thread merges, normalises and stores
  const bool cin = t0 + col < P;

  // this wave's weights: A[row l16][k 4s + kq] = W[co0 + l16][4s + kq], in
  // lane order (pack_mfma_lanes): step group j is one float4 per lane, the
  // wave's 64 of them contiguous
  const int co0 = wave * 16;
  const __amdgpu_buffer_rsrc_t wrs = uniform_rsrc(a.w, 4u * (unsigned)(C * C));
  const unsigned wof = 16u * (unsigned)(wave * (C / 16) * 64 + lane);
  float wv[C / 4];
#pragma unroll
  for (int s = 0; s < C / 16; ++s) {
    const float4 v = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(wrs, wof, 1024u * s, 0));
    wv[4 * s] = v.x;
    wv[4 * s + 1] = v.y;
    wv[4 * s + 2] = v.z;
    wv[4 * s + 3] = v.w;
  }
  // epilogue operands: rows co0 + 4 kq + g, column t0 + l16
  const __amdgpu_buffer_rsrc_t rrs = uniform_rsrc(a.res + (long long)b * C * P, 4u * (unsigned)(C * P));
  float bias[4], rv[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int co = co0 + 4 * kq + g;
    bias[g] = a.bias[co];
    rv[g] = __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(rrs, t0 + l16 < P ? 4u * (unsigned)(co * P + t0 + l16) : kBufOut,
                                                    0, 0));
  }

  // ---- the attention output tile a[C][BN] into LDS ----
  if constexpr (KSM == 1) {
    const __amdgpu_buffer_rsrc_t ars = uniform_rsrc(a.att + (long long)b * C * P, 4u * (unsigned)(C * P));
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const int ci = tid / BN + (NT / BN) * j;
      xs[tid + NT * j] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(ars, cin ? 4u * (unsigned)(ci * P + t0 + col) : kBufOut, 0, 0));
    }
  } else {
    // part[b][h][s] = (m[P], l[P], O[D][P]); slice = (D + 2) * P floats.
    // Each thread merges its own EPT elements of one column: it loads the
    // (m, l) of every split of the heads they belong to and all their O
    // values at once, then forms M = max_s m_s, f_s = e^(m_s - M) (0 for an
    // empty split, m = -inf), L = sum_s l_s f_s and O = sum_s O_s f_s in
    // split order: no LDS table, no barrier, no serial recurrence.
    const unsigned slice = (unsigned)((D + 2) * P);
    const __amdgpu_buffer_rsrc_t prs =
        uniform_rsrc(a.part + (long long)b * H * KS * slice, 4u * (unsigned)(H * KS) * slice);
    const unsigned tc = (unsigned)(t0 + col);
    float ov[EPT][KSM], mv[EPT][KSM], lv[EPT][KSM];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const int ci = tid / BN + (NT / BN) * j;
      const int h = ci / D, d = ci - h * D;
      const unsigned hb = (unsigned)(h * KS) * slice;
      const unsigned off = cin ? 4u * (hb + (unsigned)(2 + d) * P + tc) : kBufOut;
      const unsigned moff = cin ? 4u * (hb + tc) : kBufOut;
#pragma unroll
      for (int u = 0; u < KSM; ++u) {
        const unsigned su = 4u * u * slice;
        ov[j][u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(prs, u < KS ? off : kBufOut, su, 0));
        // heads change every D channels: elements of the same head reload
        // the same (m, l) words, which the cache serves
        mv[j][u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(prs, u < KS ? moff : kBufOut, su, 0));
        lv[j][u] =
            __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(prs, u < KS ? moff : kBufOut, su + 4u * P, 0));
      }
    }
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      float M = -INFINITY;
#pragma unroll
      for (int u = 0; u < KSM; ++u)
        if (u < KS) M = fmaxf(M, mv[j][u]);
      float L = 0.f, O = 0.f;
#pragma unroll
      for (int u = 0; u < KSM; ++u) {
        if (u < KS && mv[j][u] != -INFINITY) {
          const float f = expf(mv[j][u] - M);
          L = L + lv[j][u] * f;
          O = O + ov[j][u] * f;
        }
      }
      xs[tid + NT * j] = cin ? O / L : 0.f;
    }
  }
  __syncthreads();

  // ---- conv_o: rows [co0, co0 + 16) x 16 columns, the whole reduction ----
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  const float* xl = xs + kq * BN + l16;
#pragma unroll
  for (int s = 0; s < C / 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[s], xl[4 * s * BN], acc, 0, 0, 0);
  float y[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) y[g] = (acc[g] + bias[g]) + rv[g];
  __syncthreads();  // every wave has read the attention tile
#pragma unroll
  for (int g = 0; g < 4; ++g) xs[(co0 + 4 * kq + g) * BN + l16] = y[g];
  __syncthreads();

  // ---- LayerNorm over the C rows of each column ----
  constexpr int RG = NT / BN;  // row groups: thread (rg, col) takes rows rg + RG * i
  const int rg = tid / BN;
  float gv[C / RG], bv[C / RG];
#pragma unroll
  for (int i = 0; i < C / RG; ++i) {
    gv[i] = a.g[rg + RG * i];
    bv[i] = a.beta[rg + RG * i];
  }
  double sm = 0.0;
#pragma unroll
  for (int i = 0; i < C / RG; ++i) sm += xs[(rg + RG * i) * BN + col];
  red[rg][col] = sm;
  __syncthreads();
  if (tid < BN) {
    double t = 0.0;
    for (int g = 0; g < RG; ++g) t += red[g][tid];
    stat[0][tid] = (float)(t / C);
  }
  __syncthreads();
  const float mean = stat[0][col];
  double q = 0.0;
#pragma unroll
  for (int i = 0; i < C / RG; ++i) {
    const float d = xs[(rg + RG * i) * BN + col] - mean;
    q += (double)d * d;
  }
  red[rg][col] = q;
  __syncthreads();
  if (tid < BN) {
    double t = 0.0;
    for (int g = 0; g < RG; ++g) t += red[g][tid];
    stat[1][tid] = sqrtf((float)(t / C) + a.eps);
  }
  __syncthreads();
  const float den = stat[1][col];
  if (cin) {
    float* ob = a.out + (long long)b * C * P + t0 + col;
#pragma unroll
    for (int i = 0; i < C / RG; ++i) {
      const int r = rg + RG * i;
      ob[(long long)r * P] = (xs[r * BN + col] - mean) / den * gv[i] + bv[i];
    }
  }
}

template <int RT>
void launch_rt(const AttnOutArgs& a, dim3 grid, hipStream_t s) {
  if (a.KS == 1)
    hipLaunchKernelGGL((attn_out_ln_kernel<RT, 1>), grid, dim3(64 * RT), 0, s, a);
  else
    hipLaunchKernelGGL((attn_out_ln_kernel<RT, kMaxKS>), grid, dim3(64 * RT), 0, s, a);
}

}  // namespace

bool attn_out_ln_supported(int H, int D, int KS) {
  const int C = H * D;
  return H >= 1 && D >= 1 && (C == 64 || C == 96 || C == 128 || C == 192 || C == 256) && KS >= 1 && KS <= kMaxKS;
}

void launch_attn_out_ln(const AttnOutArgs& a, int B, hipStream_t s) {
  const int C = a.H * a.D;
  RVC_CHECK(attn_out_ln_supported(a.H, a.D, a.KS), "attn_out_ln: unsupported channel count or key split");
  RVC_CHECK(a.KS == 1 ? a.att != nullptr : a.part != nullptr, "attn_out_ln: missing attention input");
  RVC_CHECK(a.w && B >= 1 && a.P >= 1, "attn_out_ln: invalid shape");
  // 32-bit byte offsets: one batch item's partial slices and [C][P] tensors
  RVC_CHECK(4.0 * a.H * a.KS * (a.D + 2.0) * a.P < 2147483648.0 && 4.0 * C * a.P < 2147483648.0,
            "attn_out_ln: sequence too long for 32-bit offsets");
  const dim3 grid((unsigned)((a.P + BN - 1) / BN), (unsigned)B);
  switch (C / 16) {
    case 4: launch_rt<4>(a, grid, s); break;
    case 6: launch_rt<6>(a, grid, s); break;
    case 8: launch_rt<8>(a, grid, s); break;
    case 12: launch_rt<12>(a, grid, s); break;
    default: launch_rt<16>(a, grid, s); break;
  }
  check_launch("attn_out_ln");
}

}  // namespace rvc
