// Windowed relative-position self-attention of enc_p (VITS T5-style, window
// w = 10) as fused fp32 MFMA kernels, flash style: no [H,P,P] score tensor
// and none of the [H,P,2P-1] rel/abs tensors the numpy path builds
// (runtime/models/vits.py:994-1016).
//
//   qs_t       = q_t / sqrt(D)
//   score[t,s] = qs_t . k_s  +  [|s-t| <= w] qs_t . emb_k[s-t+w]
//   p[t,:]     = softmax(score[t,:])
//   out_t      = sum_s p[t,s] v_s  +  sum_{|s-t|<=w} p[t,s] emb_v[s-t+w]
//
// emb_rel is zero outside the window after _get_relative_embeddings
// (runtime/models/vits.py:448-462), so only the 2w+1 band diagonals carry the
// relative terms.  With emb_k == emb_v == null the band terms vanish and the
// kernel is plain scaled-dot-product attention (HuBERT's self-attention,
// q scaled by 1/sqrt(D), runtime/models/hubert.py:1315-1338).
//
// A workgroup owns 32 queries of one head and one slice of the keys (the key
// axis is split over KS workgroups so short sequences still fill the GPU);
// its 4 waves take every 4th 32-key tile of the slice and keep their own
// running max / sum / output (online softmax), merged through LDS.  With
// KS > 1 the slices' partial (max, sum, output) go to a scratch buffer and a
// second kernel merges them.
//
// Per key tile a wave computes S^T = K_tile^T Q with v_mfma_f32_32x32x2_f32
// (rows = keys in registers, columns = queries in lanes), so the per-query
// softmax statistics are a reduction over the lane's own registers plus one
// swap with the other half-wave, and the probabilities already sit in the
// B-operand layout of O^T += V P^T: MFMA step r pairs key rows (r%4)+8*(r/4)
// and (r%4)+4+8*(r/4), exactly the rows accumulator register r holds in the
// two half-waves.  The band terms: R^T[r][t] = emb_k[r] . qs_t is one extra
// MFMA tile added to the in-band scores; the in-band probabilities are
// collected per wave ([2w+1][32], rescaled with the running max) and
// contracted with emb_v by MFMA after the key loop.
#include <algorithm>

#include "internal.h"

namespace rvc {

typedef float floatx16 __attribute__((ext_vector_type(16)));

namespace {

constexpr int AWAVES = 4;
constexpr int kMaxWindow = 15;  // 2w+1 <= 31 band rows fit one 32-row tile

__device__ __forceinline__ int acc_row(int r, int half) { return (r & 3) + 4 * half + 8 * (r >> 2); }

template <int DT>
struct AttnLds {
  static constexpr int ROWS = DT * 32;
  static constexpr int VSTRIDE = 33;
  static constexpr int Q = ROWS * 32;                  // qs[d][t]
  static constexpr int V = AWAVES * ROWS * VSTRIDE;    // per-wave V tiles
  static constexpr int MERGE = (AWAVES - 1) * (DT * 16 * 64 + 2 * 32);
  static constexpr int R = 32 * 32;                    // R^T[r][t]
  static constexpr int VM = V > MERGE ? V : MERGE;
  // then per wave the band probabilities [r][t], rows [0, nb) and a junk row nb
  static size_t bytes(int nb) { return sizeof(float) * (Q + VM + R + AWAVES * (nb + 1) * 32); }
};

// DT <= 2 (HuBERT's 64-wide heads) is held to three waves per SIMD (at most
// 168 registers): three workgroups per CU, which sets the key split (4 at
// 499 frames, 16.2 us per layer, against 3 splits and 21 us at two per CU).
template <int DT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DT <= 2 ? 3 : 1))) void relpos_attention_kernel(const float* qkv, const float* emb_k,
                                                               const float* emb_v, float* out, float* part, int H,
                                                               int D, int P, int window, int KS) {
  using Lds = AttnLds<DT>;
  constexpr int NKK = DT * 16;
  extern __shared__ float sm[];
  float* Qs = sm;
  float* VM = sm + Lds::Q;
  float* Rl = VM + Lds::VM;
  float* PbAll = Rl + Lds::R;

  const int h = blockIdx.y;
  const int b = blockIdx.z / KS;
  const int ks = blockIdx.z - b * KS;
  const int t0 = blockIdx.x * 32;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const long long CP = (long long)H * D * P;
  const float* qb = qkv + (long long)b * 3 * CP + (long long)h * D * P;
  // one buffer resource per operand block ([D][P] each); masked lanes read 0
  const unsigned blk = 4u * (unsigned)(D * P);
  const __amdgpu_buffer_rsrc_t qrs = uniform_rsrc(qb, blk);
  const __amdgpu_buffer_rsrc_t krs = uniform_rsrc(qb + CP, blk);
  const __amdgpu_buffer_rsrc_t vrs = uniform_rsrc(qb + 2 * CP, blk);
  const int nb = emb_k != nullptr ? 2 * window + 1 : 0;  // no band: plain attention
  const int t = t0 + l32;
  const float sq = sqrtf((float)D);
  // this workgroup's key tiles [kt_begin, kt_end); the band rows are needed
  // only where the slice meets keys [t0 - window, t0 + 31 + window]
  const int ntile = (P + 31) / 32;
  const int per = (ntile + KS - 1) / KS;
  const int kt_begin = ks * per;
  const int kt_end = min(ntile, (ks + 1) * per);
  const bool slice_near = nb > 0 && kt_begin * 32 <= t0 + 31 + window && kt_end * 32 - 1 >= t0 - window;

  // stage qs[d][t] = q[d][t0 + t] / sqrt(D): every load in flight before
  // the first division (a rolled loop waits out one round trip per element)
  {
    constexpr int QPT = Lds::Q / 256;
    static_assert(Lds::Q % 256 == 0, "whole staging rounds");
    float qv[QPT];
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const int e = tid + 256 * i;
      const int d = e >> 5, j = e & 31;
      const unsigned off = (d < D && t0 + j < P) ? 4u * (unsigned)(d * P + t0 + j) : kBufOut;
      qv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(qrs, off, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < QPT; ++i) Qs[tid + 256 * i] = qv[i] / sq;
  }
  // band probabilities per wave: rows [0, nb) live, row nb takes the masked
  // lanes' (zero) updates so every lane can store unconditionally
  float* Pb = PbAll + wave * (nb + 1) * 32;
  for (int e = lane; e < (nb + 1) * 32; e += 64) Pb[e] = 0.f;
  __syncthreads();
  // R^T[r][t] = emb_k[r] . qs_t   (wave 0)
  if (wave == 0 && slice_near) {
    const __amdgpu_buffer_rsrc_t ers = uniform_rsrc(emb_k, 4u * (unsigned)(nb * D));
    floatx16 racc;
#pragma unroll
    for (int r = 0; r < 16; ++r) racc[r] = 0.f;
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
      const int d = 2 * kk + half;
      const unsigned off = (l32 < nb && d < D) ? 4u * (unsigned)(l32 * D + d) : kBufOut;
      const float a = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ers, off, 0, 0));
      racc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, Qs[d * 32 + l32], racc, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) Rl[acc_row(r, half) * 32 + l32] = racc[r];
  }
  __syncthreads();

  float* Vt = VM + wave * Lds::ROWS * Lds::VSTRIDE;
  floatx16 O[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) O[dt][r] = 0.f;
  float m = -INFINITY;  // running max of query t (same in both half-waves)
  float l = 0.f;        // running sum over this half-wave's key rows
  bool band_seen = false;  // wave-uniform: Pb holds probabilities to rescale

  for (int kt = kt_begin + wave; kt < kt_end; kt += AWAVES) {
    const int s0 = kt * 32;
    // all global loads of the tile first: K operands and the V tile
    // K operand kk and V staging element i read the same lane position:
    // row 2 * kk + half (2 * i + half), key s0 + l32.  Rows at or past D fall
    // outside the [D][P] block and read 0; a key past P takes an offset above
    // every range (kBufOut + at most 63 row steps stays below 2^32, the
    // launcher bounds P).
    const unsigned base = s0 + l32 < P ? 4u * (unsigned)(half * P + s0 + l32) : kBufOut;
    const unsigned rstep = 8u * (unsigned)P;
    float kreg[NKK];
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk)
      kreg[kk] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(krs, base + kk * rstep, 0, 0));
    float vreg[DT * 16];
#pragma unroll
    for (int i = 0; i < DT * 16; ++i)
      vreg[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(vrs, base + i * rstep, 0, 0));
    // S^T[s][t] = sum_d k[d][s] qs[d][t]
    floatx16 S;
#pragma unroll
    for (int r = 0; r < 16; ++r) S[r] = 0.f;
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk)
      S = __builtin_amdgcn_mfma_f32_32x32x2f32(kreg[kk], Qs[(2 * kk + half) * 32 + l32], S, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < DT * 16; ++i) {
      const int e = lane + 64 * i;
      Vt[(e >> 5) * Lds::VSTRIDE + (e & 31)] = vreg[i];
    }
    // band terms (wave-uniform test) and key mask
    const bool near = nb > 0 && s0 <= t0 + 31 + window && s0 + 31 >= t0 - window;
    if (near) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int rr = s0 + acc_row(r, half) - t + window;
        const bool in = (unsigned)rr < (unsigned)nb;
        const float rv = Rl[(in ? rr : 0) * 32 + l32];
        S[r] = in ? S[r] + rv : S[r];
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) S[r] = s0 + acc_row(r, half) < P ? S[r] : -INFINITY;
    // online softmax statistics of query t
    float tm = S[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) tm = fmaxf(tm, S[r]);
    tm = fmaxf(tm, __shfl_xor(tm, 32));
    const float m_new = fmaxf(m, tm);
    const float alpha = expf(m - m_new);
    float sum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = expf(S[r] - m_new);
      S[r] = p;
      sum += p;
    }
    l = l * alpha + sum;
    m = m_new;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) O[dt][r] *= alpha;
    if (band_seen) {
      // the two half-waves rescale rows [0, 16) and [16, nb)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (16 * half + i < nb) Pb[(16 * half + i) * 32 + l32] *= alpha;
    }
    if (near) {
      band_seen = true;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int rr = s0 + acc_row(r, half) - t + window;
        const bool in = (unsigned)rr < (unsigned)nb;
        float* pe = Pb + (in ? rr : nb) * 32 + l32;
        *pe = *pe + (in ? S[r] : 0.f);
      }
    }
    // O^T[d][t] += sum_s V[d][s] P^T[s][t]
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const float* vrow = Vt + (dt * 32 + l32) * Lds::VSTRIDE;
#pragma unroll
      for (int r = 0; r < 16; ++r)
        O[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[acc_row(r, half)], S[r], O[dt], 0, 0, 0);
    }
  }

  // band contribution: O^T[d][t] += sum_r emb_v[r][d] Pb[r][t].  emb_v
  // ([nb][D], nb * D < Lds::Q) goes through LDS, into the query tile's
  // region once every wave has left the key loop, with all its loads in
  // flight; a wave that saw the band lies in a slice that meets it.
  if (slice_near) {  // uniform for the workgroup
    __syncthreads();  // the query tile is dead
    constexpr int QPT = Lds::Q / 256;
    const int nv = nb * D;
    const __amdgpu_buffer_rsrc_t ers = uniform_rsrc(emb_v, 4u * (unsigned)nv);
    float ev[QPT];
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const int e = tid + 256 * i;
      ev[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ers, e < nv ? 4u * (unsigned)e : kBufOut, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < QPT; ++i)
      if (tid + 256 * i < nv) Qs[tid + 256 * i] = ev[i];
    __syncthreads();
  }
  if (band_seen) {
    for (int kk = 0; kk < (nb + 1) / 2; ++kk) {
      const int rr = 2 * kk + half;
      const float bval = Pb[rr * 32 + l32];  // row nb (odd nb) stays zero
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int d = dt * 32 + l32;
        const float a = (rr < nb && d < D) ? Qs[rr * D + d] : 0.f;
        O[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, bval, O[dt], 0, 0, 0);
      }
    }
  }
  l = l + __shfl_xor(l, 32);

  // merge the four waves: M = max m_w, L = sum l_w e^(m_w-M), O = sum O_w e^(m_w-M)
  __syncthreads();  // V tiles are dead; reuse their LDS for the merge
  constexpr int PER = DT * 16 * 64 + 2 * 32;
  if (wave > 0) {
    float* dst = VM + (wave - 1) * PER;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) dst[(dt * 16 + r) * 64 + lane] = O[dt][r];
    if (half == 0) {
      dst[DT * 16 * 64 + l32] = m;
      dst[DT * 16 * 64 + 32 + l32] = l;
    }
  }
  __syncthreads();
  if (wave > 0) return;
  float M = m;
  for (int w = 1; w < AWAVES; ++w) M = fmaxf(M, VM[(w - 1) * PER + DT * 16 * 64 + l32]);
  // a slice with no keys at all keeps M = -inf; its partial carries zero weight
  const float f0 = M == -INFINITY ? 0.f : expf(m - M);
  float L = l * f0;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) O[dt][r] *= f0;
  for (int w = 1; w < AWAVES; ++w) {
    const float* src = VM + (w - 1) * PER;
    const float mw = src[DT * 16 * 64 + l32];
    const float f = M == -INFINITY ? 0.f : expf(mw - M);
    L += src[DT * 16 * 64 + 32 + l32] * f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) O[dt][r] += src[(dt * 16 + r) * 64 + lane] * f;
  }
  if (t >= P) return;
  if (KS == 1) {
    float* ob = out + (long long)b * H * D * P + (long long)h * D * P;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = dt * 32 + acc_row(r, half);
        if (d < D) ob[(long long)d * P + t] = O[dt][r] / L;
      }
  } else {
    // partial slice: part[((b*H + h)*KS + ks)] holds m[P], l[P], O[D][P]
    float* pb = part + ((long long)(b * H + h) * KS + ks) * (long long)(D + 2) * P;
    if (half == 0) {
      pb[t] = M;
      pb[P + t] = L;
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = dt * 32 + acc_row(r, half);
        if (d < D) pb[(long long)(2 + d) * P + t] = O[dt][r];
      }
  }
}

// out[b][h*D+d][t] = sum_ks O_ks e^(m_ks - M) / sum_ks l_ks e^(m_ks - M), M the
// largest m_ks: one pass over the slices with a running maximum (an empty
// slice, m = -inf, carries no weight)
__global__ __launch_bounds__(256) void relpos_attention_merge(const float* part, float* out, int H, int D, int P,
                                                              int KS, long long n) {
  const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
  if (e >= n) return;
  const int t = (int)(e % P);
  const long long r = e / P;
  const int d = (int)(r % D);
  const long long bh = r / D;
  const long long slice = (long long)(D + 2) * P;
  const float* pb = part + bh * KS * slice;
  constexpr int U = 8;  // slices whose loads are in flight together
  float M = -INFINITY, L = 0.f, O = 0.f;
  for (int k0 = 0; k0 < KS; k0 += U) {
    float mk[U], lk[U], ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float* s = pb + min(k0 + u, KS - 1) * slice;  // past KS: re-reads the last slice, skipped below
      mk[u] = s[t];
      lk[u] = s[P + t];
      ok[u] = s[(long long)(2 + d) * P + t];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (k0 + u >= KS || mk[u] == -INFINITY) continue;
      const float Mn = fmaxf(M, mk[u]);
      const float fo = expf(M - Mn);  // 0 while M = -inf
      const float fk = expf(mk[u] - Mn);
      L = L * fo + lk[u] * fk;
      O = O * fo + ok[u] * fk;
      M = Mn;
    }
  }
  out[(bh * D + d) * (long long)P + t] = O / L;
}

template <int DT>
void launch_dt(const float* qkv, const float* emb_k, const float* emb_v, float* out, float* part, int B, int H,
               int D, int P, int window, int KS, hipStream_t s) {
  const int nb = emb_k != nullptr ? 2 * window + 1 : 0;
  const size_t lds = AttnLds<DT>::bytes(nb);
  static bool attr = false;
  if (!attr) {
    RVC_HIP(hipFuncSetAttribute((const void*)relpos_attention_kernel<DT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)AttnLds<DT>::bytes(2 * kMaxWindow + 1)));
    attr = true;
  }
  dim3 grid((P + 31) / 32, H, B * KS);
  hipLaunchKernelGGL(relpos_attention_kernel<DT>, grid, dim3(256), lds, s, qkv, emb_k, emb_v, out, part, H, D, P,
                     window, KS);
  check_launch("relpos_attention");
}

template <int DT>
int blocks_per_cu(int nb) {
  int n = 0;
  RVC_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, relpos_attention_kernel<DT>, 256, AttnLds<DT>::bytes(nb)));
  return std::max(n, 1);
}

// workgroups of the attention kernel one CU holds at once (registers and LDS)
// times the CUs, for head dim D and nb band rows
int attention_resident_blocks(int D, int nb) {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0;
    RVC_HIP(hipGetDevice(&dev));
    RVC_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  }
  switch ((D + 31) / 32) {
    case 1: return cus * blocks_per_cu<1>(nb);
    case 2: return cus * blocks_per_cu<2>(nb);
    case 3: return cus * blocks_per_cu<3>(nb);
    default: return cus * blocks_per_cu<4>(nb);
  }
}

}  // namespace

// The key split fills what the GPU holds at once (all CUs times the
// workgroups one CU takes), each wave keeping at least one key tile.  It
// depends on (H, D, P, window) only, never on B: the merge order of the split
// partial sums is part of the result's rounding, so a batched call must use
// the split a single chunk would, or batch != per-chunk bit for bit.
int relpos_attention_splits(int H, int D, int P, int window, bool band) {
  const int nb = band ? 2 * window + 1 : 0;
  const int per_gpu = attention_resident_blocks(D, nb);
  const int ntile = (P + 31) / 32;
  const int blocks = ntile * H;
  int ks = (per_gpu + blocks - 1) / blocks;
  ks = std::min(ks, std::max(1, ntile / AWAVES));
  return std::max(ks, 1);
}

size_t relpos_attention_scratch_floats(int B, int H, int D, int P, int window, bool band) {
  const int ks = relpos_attention_splits(H, D, P, window, band);
  return ks > 1 ? (size_t)B * H * ks * (D + 2) * P : 0;
}

size_t relpos_attention_max_frames() { return (size_t)1 << 30; }

int launch_relpos_attention_partials(const float* qkv, const float* emb_k, const float* emb_v, float* out,
                                     float* scratch, size_t scratch_floats, int B, int H, int D, int P, int window,
                                     hipStream_t s) {
  RVC_CHECK(D >= 1 && D <= 128, "relpos_attention: head dim must be in [1,128]");
  RVC_CHECK(window >= 0 && window <= kMaxWindow, "relpos_attention: window must be in [0,15]");
  RVC_CHECK((emb_k == nullptr) == (emb_v == nullptr), "relpos_attention: emb_k and emb_v go together");
  RVC_CHECK(P >= 1 && B >= 1 && H >= 1, "relpos_attention: invalid shape");
  // 32-bit buffer offsets: one [D][P] operand block, and the masked-key
  // offset plus 63 row steps of 2P floats, stay below 2^31 / 2^32
  RVC_CHECK((long long)D * P * 4 < (1LL << 31) && 63LL * 8 * P < (1LL << 31),
            "relpos_attention: sequence too long for 32-bit offsets");
  const int KS = relpos_attention_splits(H, D, P, window, emb_k != nullptr);
  RVC_CHECK(KS == 1 || scratch != nullptr, "relpos_attention: scratch buffer required");
  // the split partials fill B*H*KS*(D+2)*P floats of scratch
  RVC_CHECK(KS == 1 || scratch_floats >= (size_t)B * H * KS * (D + 2) * P,
            "relpos_attention: scratch buffer smaller than the key split's partial sums");
  const int dt = (D + 31) / 32;
  if (dt == 1) launch_dt<1>(qkv, emb_k, emb_v, out, scratch, B, H, D, P, window, KS, s);
  else if (dt == 2) launch_dt<2>(qkv, emb_k, emb_v, out, scratch, B, H, D, P, window, KS, s);
  else if (dt == 3) launch_dt<3>(qkv, emb_k, emb_v, out, scratch, B, H, D, P, window, KS, s);
  else launch_dt<4>(qkv, emb_k, emb_v, out, scratch, B, H, D, P, window, KS, s);
  return KS;
}

void launch_relpos_attention(const float* qkv, const float* emb_k, const float* emb_v, float* out, float* scratch,
                             size_t scratch_floats, int B, int H, int D, int P, int window, hipStream_t s) {
  const int KS =
      launch_relpos_attention_partials(qkv, emb_k, emb_v, out, scratch, scratch_floats, B, H, D, P, window, s);
  if (KS > 1) {
    const long long n = (long long)B * H * D * P;
    hipLaunchKernelGGL(relpos_attention_merge, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, scratch, out, H, D,
                       P, KS, n);
    check_launch("relpos_attention_merge");
  }
}

}  // namespace rvc
