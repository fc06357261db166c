// Windowed relative-position self-attention of enc_p (VITS T5-style, window
// w = 10), fused: scores, band terms, softmax and the weighted sums run in
// one kernel without materialising the [H,P,P] or [H,P,2P-1] tensors the
// numpy path builds (runtime/models/vits.py:994-1016).
//
//   qs_t       = q_t / sqrt(D)
//   score[t,s] = qs_t . k_s  +  [|s-t| <= w] qs_t . emb_k[s-t+w]
//   p[t,:]     = softmax(score[t,:])
//   out_t      = sum_s p[t,s] v_s  +  sum_{|s-t|<=w} p[t,s] emb_v[s-t+w]
//
// emb_rel is zero outside the window after _get_relative_embeddings
// (runtime/models/vits.py:448-462), so only the 2w+1 band diagonals carry
// the relative terms.  One workgroup handles TQ query rows of one head; the
// full score rows live in LDS.
#include "internal.h"

namespace rvc {
namespace {

constexpr int TQ = 8;
constexpr int DMAX = 128;
constexpr size_t kLdsMax = 65536;

__global__ __launch_bounds__(256) void relpos_attention_kernel(const float* qkv, const float* emb_k,
                                                               const float* emb_v, float* out, int H, int D,
                                                               int P, int window) {
  extern __shared__ float sm[];
  float* qs = sm;              // [TQ][D]
  float* S = sm + TQ * DMAX;   // [TQ][P]

  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int t0 = blockIdx.x * TQ;
  const int tid = threadIdx.x;
  const long long CP = (long long)H * D * P;
  const float* qb = qkv + (long long)b * 3 * CP + (long long)h * D * P;
  const float* kb = qb + CP;
  const float* vb = qb + 2 * CP;
  const float sq = sqrtf((float)D);

  for (int e = tid; e < TQ * D; e += 256) {
    const int tq = e / D, d = e - tq * D;
    const int t = t0 + tq;
    qs[tq * DMAX + d] = (t < P) ? qb[(long long)d * P + t] / sq : 0.f;
  }
  __syncthreads();

  // scores
  for (int s = tid; s < P; s += 256) {
    float acc[TQ];
#pragma unroll
    for (int tq = 0; tq < TQ; ++tq) acc[tq] = 0.f;
    for (int d = 0; d < D; ++d) {
      const float kv = kb[(long long)d * P + s];
#pragma unroll
      for (int tq = 0; tq < TQ; ++tq) acc[tq] += qs[tq * DMAX + d] * kv;
    }
#pragma unroll
    for (int tq = 0; tq < TQ; ++tq) {
      const int r = s - (t0 + tq);
      if (r >= -window && r <= window) {
        const float* e = emb_k + (long long)(r + window) * D;
        float a2 = 0.f;
        for (int d = 0; d < D; ++d) a2 += qs[tq * DMAX + d] * e[d];
        acc[tq] = acc[tq] + a2;
      }
      S[tq * P + s] = acc[tq];
    }
  }
  __syncthreads();

  // softmax, two query rows per wave
  const int wave = tid >> 6, lane = tid & 63;
  for (int tq = wave; tq < TQ; tq += 4) {
    float* row = S + tq * P;
    float m = -INFINITY;
    for (int s = lane; s < P; s += 64) m = fmaxf(m, row[s]);
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    float sum = 0.f;
    for (int s = lane; s < P; s += 64) {
      const float e = expf(row[s] - m);
      row[s] = e;
      sum += e;
    }
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
    for (int s = lane; s < P; s += 64) row[s] = row[s] / sum;
  }
  __syncthreads();

  // weighted sums
  for (int e = tid; e < TQ * D; e += 256) {
    const int tq = e / D, d = e - tq * D;
    const int t = t0 + tq;
    if (t >= P) continue;
    const float* row = S + tq * P;
    const float* vr = vb + (long long)d * P;
    float acc = 0.f;
    for (int s = 0; s < P; ++s) acc += row[s] * vr[s];
    float a2 = 0.f;
    const int s_lo = max(0, t - window), s_hi = min(P - 1, t + window);
    for (int s = s_lo; s <= s_hi; ++s) a2 += row[s] * emb_v[(long long)(s - t + window) * D + d];
    out[(long long)b * H * D * P + (long long)(h * D + d) * P + t] = acc + a2;
  }
}

}  // namespace

size_t relpos_attention_max_frames() { return (kLdsMax / sizeof(float) - TQ * DMAX) / TQ; }

void launch_relpos_attention(const float* qkv, const float* emb_k, const float* emb_v, float* out, int B,
                             int H, int D, int P, int window, hipStream_t s) {
  RVC_CHECK(D >= 1 && D <= DMAX, "relpos_attention: head dim must be in [1,128]");
  RVC_CHECK(P >= 1 && (size_t)P <= relpos_attention_max_frames(),
            "relpos_attention: too many frames for the LDS score rows");
  const size_t lds = sizeof(float) * ((size_t)TQ * DMAX + (size_t)TQ * P);
  dim3 grid((P + TQ - 1) / TQ, H, B);
  hipLaunchKernelGGL(relpos_attention_kernel, grid, dim3(256), lds, s, qkv, emb_k, emb_v, out, H, D, P,
                     window);
  check_launch("relpos_attention");
}

}  // namespace rvc
