// Kernels of the glue around synthesis (runtime/pipeline.py): feature
// retrieval (brute-force L2 k-nearest neighbours and the (1/d)^2 blend), the
// 2x linear interpolation of the features with the pitch protect mask, the RMS
// envelope mix and the int16 peak normalisation.
//
// The float32 expressions and their evaluation order follow the reference's
// numpy code line by line (contraction into fused multiply-adds is off), so
// every elementwise result is bit-identical to it; the only differences come
// from summation order inside the distance dot products (an MFMA GEMM) and the
// squared norms / RMS frame sums (fixed reduction trees here, numpy's pairwise
// sums there).
#include <cfloat>
#include <climits>

#include "internal.h"

namespace rvc {

namespace {

constexpr int kTopK = 8;  // the pipeline searches k = 8 (runtime/pipeline.py:55)

// out[r] = sum_c x[r][c]^2, one wave per row (lane-strided partial sums, then
// a fixed butterfly across the wave).
__global__ __launch_bounds__(256) void row_sqnorm_kernel(const float* x, float* out, long long rows, int cols) {
#pragma clang fp contract(off)
  const long long r = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const float* p = x + r * cols;
  float s = 0.f;
  for (int c = lane; c < cols; c += 64) s = s + p[c] * p[c];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s = s + __shfl_xor(s, o);
  if (lane == 0) out[r] = s;
}

// Keep the kTopK smallest (distance, row) pairs in lexicographic order:
// among equal distances the lower row ranks first, whatever order the
// candidates arrive in (a NaN distance compares false and is never kept).
__device__ __forceinline__ bool lex_less(float d, int n, float bd, int bn) { return d < bd || (d == bd && n < bn); }
__device__ __forceinline__ void topk_insert(float (&bs)[kTopK], int (&bi)[kTopK], float d, int n) {
  if (!lex_less(d, n, bs[kTopK - 1], bi[kTopK - 1])) return;
#pragma unroll
  for (int j = 0; j < kTopK; ++j) {
    const bool sw = lex_less(d, n, bs[j], bi[j]);
    const float tb = bs[j];
    const int ti = bi[j];
    bs[j] = sw ? d : tb;
    bi[j] = sw ? n : ti;
    d = sw ? tb : d;
    n = sw ? ti : n;
  }
}

// Partial top-k of one slice of database rows for 64 queries (one per lane):
// dist = (q2[f] + d2[n]) - 2 * dot[n][f], clamped at 0
// (runtime/retrieval.py:56-62).  Writes [slice][F][kTopK].
__global__ __launch_bounds__(64) void knn_partial_kernel(const float* dot, long long ldd, const float* q2,
                                                         const float* d2, int F, int N, int per, float* ps, int* pi) {
#pragma clang fp contract(off)
  const int f = blockIdx.x * 64 + threadIdx.x;
  const int s = blockIdx.y;
  const int n0 = s * per;
  const int n1 = min(N, n0 + per);
  float bs[kTopK];
  int bi[kTopK];
#pragma unroll
  for (int j = 0; j < kTopK; ++j) {
    bs[j] = INFINITY;
    bi[j] = INT_MAX;
  }
  if (f < F) {
    const float qq = q2[f];
    auto dist = [&](float dd, float v) {
      const float d = (qq + dd) - 2.0f * v;
      return d < 0.f ? 0.f : d;  // np.maximum(dist, 0): a NaN stays NaN and is never kept
    };
    // blocks of 16 rows: the 16 loads are issued before any is consumed
    int n = n0;
    for (; n + 16 <= n1; n += 16) {
      float v[16], dd[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        v[u] = dot[(long long)(n + u) * ldd + f];
        dd[u] = d2[n + u];
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) topk_insert(bs, bi, dist(dd[u], v[u]), n + u);
    }
    for (; n < n1; ++n) topk_insert(bs, bi, dist(d2[n], dot[(long long)n * ldd + f]), n);
    const long long o = ((long long)s * F + f) * kTopK;
#pragma unroll
    for (int j = 0; j < kTopK; ++j) {
      ps[o + j] = bs[j];
      pi[o + j] = bi[j];
    }
  }
}

// Merge the slices' partial lists of each query, one wave per query: lane l
// folds slices l, l+64, ... into its own list, then a butterfly over the
// wave merges the 64 lists (every lane ends with the full top list); the
// first k entries go to scores [F][k] / indices [F][k] (int64).
__global__ __launch_bounds__(256) void knn_merge_kernel(const float* ps, const int* pi, int F, int S, int k,
                                                        float* scores, long long* inds) {
  const int f = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (f >= F) return;  // whole waves
  float bs[kTopK];
  int bi[kTopK];
#pragma unroll
  for (int j = 0; j < kTopK; ++j) {
    bs[j] = INFINITY;
    bi[j] = INT_MAX;
  }
  for (int s = lane; s < S; s += 64) {
    const long long o = ((long long)s * F + f) * kTopK;
    float cs[kTopK];
    int ci[kTopK];
#pragma unroll
    for (int j = 0; j < kTopK; ++j) {
      cs[j] = ps[o + j];
      ci[j] = pi[o + j];
    }
#pragma unroll
    for (int j = 0; j < kTopK; ++j) topk_insert(bs, bi, cs[j], ci[j]);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    float os[kTopK];
    int oi[kTopK];
#pragma unroll
    for (int j = 0; j < kTopK; ++j) {
      os[j] = __shfl_xor(bs[j], off);
      oi[j] = __shfl_xor(bi[j], off);
    }
#pragma unroll
    for (int j = 0; j < kTopK; ++j) topk_insert(bs, bi, os[j], oi[j]);
  }
  if (lane < k) {
    // lane j writes entry j (registers indexed by a compile-time j)
#pragma unroll
    for (int j = 0; j < kTopK; ++j)
      if (j == lane) {
        scores[(long long)f * k + j] = bs[j];
        inds[(long long)f * k + j] = bi[j] == INT_MAX ? -1 : bi[j];
      }
  }
}

// Retrieval blend of runtime/pipeline.py:546-566 (FeatureIndex branch, brute
// mix 0): w = (1/score)^2, w /= max(sum w, 1e-12), blend = sum_j vecs[ix_j] w_j,
// blend = (1 - 0) * blend + 0 * blend, feats = blend * rate + feats * (1 - rate).
// One thread per (query, dim).  The row sum follows numpy's reduction of
// k = 8 contiguous values ((w0+w1)+(w2+w3)) + ((w4+w5)+(w6+w7)) and a plain
// left-to-right sum below 8; the sum over neighbours runs left to right.
__global__ __launch_bounds__(256) void retrieval_blend_kernel(const float* scores, const long long* inds,
                                                              const float* vecs, const float* feats, float* out,
                                                              int F, int D, int N, int k, float rate, float omr) {
#pragma clang fp contract(off)
  const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
  if (e >= (long long)F * D) return;
  const int f = (int)(e / D);
  const int d = (int)(e - (long long)f * D);
  float w[kTopK];
#pragma unroll
  for (int j = 0; j < kTopK; ++j) {
    if (j < k) {
      const float r = 1.0f / scores[(long long)f * k + j];
      w[j] = r * r;
    } else {
      w[j] = 0.f;
    }
  }
  float sum;
  if (k == kTopK) {
    sum = ((w[0] + w[1]) + (w[2] + w[3])) + ((w[4] + w[5]) + (w[6] + w[7]));
  } else {
    sum = 0.f;
#pragma unroll
    for (int j = 0; j < kTopK; ++j)
      if (j < k) sum = sum + w[j];
  }
  const float den = fmaxf(sum, 1e-12f);
  float b = 0.f;
#pragma unroll
  for (int j = 0; j < kTopK; ++j) {
    if (j < k) {
      // a neighbour slot left empty (only when distances were NaN) reads NaN
      const long long r = inds[(long long)f * k + j];
      const float v = r >= 0 && r < N ? vecs[r * (long long)D + d] : __builtin_nanf("");
      const float p = v * (w[j] / den);
      b = j == 0 ? p : b + p;
    }
  }
  b = b * 1.0f + b * 0.0f;
  out[e] = b * rate + feats[e] * omr;
}

// 2x linear interpolation along time of x[F][D] -> [2F][D]
// (runtime/nn.py:734-758 with scale 2: src = (i + 0.5) / 2 - 0.5 clamped to
// [0, F-1], frac cast to float32), then, when pitchf is given, the protect mask
// of runtime/pipeline.py:595-610: pff = 1 where pitchf > 0, protect where
// pitchf < 1 (in that order), out = a * pff + a0 * (1 - pff) with a0 the same
// interpolation of x0.
__global__ __launch_bounds__(256) void interp2_protect_kernel(const float* x, const float* x0, const float* pitchf,
                                                              float protect, float* out, int F, int D) {
#pragma clang fp contract(off)
  const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
  if (e >= 2LL * F * D) return;
  const int i = (int)(e / D);
  const int d = (int)(e - (long long)i * D);
  double src = ((double)i + 0.5) / 2.0 - 0.5;
  src = fmin(fmax(src, 0.0), (double)(F - 1));
  const int lo = (int)floor(src);
  const int hi = min(lo + 1, F - 1);
  const float fr = (float)(src - (double)lo);
  const float a = x[(long long)lo * D + d] * (1.0f - fr) + x[(long long)hi * D + d] * fr;
  if (!pitchf) {
    out[e] = a;
    return;
  }
  const float a0 = x0[(long long)lo * D + d] * (1.0f - fr) + x0[(long long)hi * D + d] * fr;
  const float pf = pitchf[i];
  float pff = pf;
  if (pf > 0.f) pff = 1.0f;
  if (pf < 1.f) pff = protect;
  out[e] = a * pff + a0 * (1.0f - pff);
}

// RMS of each half-second frame (runtime/pipeline.py:191-206, librosa rms with
// center=True and zero padding): frame t covers x[t*hop - hop, t*hop + hop),
// frame length 2*hop.  One workgroup per frame; float32 partial sums in a
// fixed tree, mean = sum / frame_length, then sqrt.
__global__ __launch_bounds__(256) void rms_frames_kernel(const float* x, long long n, int hop, float* out) {
#pragma clang fp contract(off)
  __shared__ float red[256];
  const long long t = blockIdx.x;
  const long long fl = 2LL * hop;
  const long long start = t * hop - hop;
  float s = 0.f;
  for (long long j = threadIdx.x; j < fl; j += 256) {
    const long long q = start + j;
    if (q >= 0 && q < n) {
      const float v = x[q];
      s = s + v * v;
    }
  }
  red[threadIdx.x] = s;
  __syncthreads();
  for (int o = 128; o >= 1; o >>= 1) {
    if ((int)threadIdx.x < o) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[t] = sqrtf(red[0] / (float)fl);
}

// Linear interpolation of r[L] onto n_out points in float64
// (runtime/pipeline.py:209-232), returned as float32.
__device__ __forceinline__ float interp_size(const float* r, int L, long long i, long long n_out) {
#pragma clang fp contract(off)
  if (L == n_out) return r[i];
  double src = ((double)i + 0.5) * ((double)L / (double)n_out) - 0.5;
  src = fmin(fmax(src, 0.0), (double)(L - 1));
  const long long lo = (long long)floor(src);
  const long long hi = lo + 1 < L - 1 ? lo + 1 : L - 1;
  const double fr = src - (double)lo;
  return (float)((double)r[lo] * (1.0 - fr) + (double)r[hi] * fr);
}

// data2 * pow(r1, 1 - rate) * pow(max(r2, 1e-6), rate - 1) with r1, r2 the
// frame RMS curves interpolated to len(data2) (runtime/pipeline.py:164-188).
__global__ __launch_bounds__(256) void rms_mix_kernel(const float* data2, long long n2, const float* r1, int L1,
                                                      const float* r2, int L2, float e1, float e2, float* out) {
#pragma clang fp contract(off)
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n2) return;
  const float a = interp_size(r1, L1, i, n2);
  const float b = fmaxf(interp_size(r2, L2, i, n2), 1e-6f);
  const float ratio = powf(a, e1) * powf(b, e2);
  out[i] = data2[i] * ratio;
}

// max |x| over n values: per-workgroup maxima (order-free, exact), then one
// workgroup folds them.
__global__ __launch_bounds__(256) void absmax_kernel(const float* x, long long n, float* part) {
  __shared__ float red[256];
  float m = 0.f;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)gridDim.x * 256)
    m = fmaxf(m, fabsf(x[i]));
  red[threadIdx.x] = m;
  __syncthreads();
  for (int o = 128; o >= 1; o >>= 1) {
    if ((int)threadIdx.x < o) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + o]);
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

// out = int16(x * scale) with scale = 32768 / (max|x| / 0.99) when that exceeds
// 1, else 32768 (runtime/pipeline.py:1208-1213; float32 arithmetic, the
// conversion truncates toward zero like numpy's astype).
__global__ __launch_bounds__(256) void to_int16_kernel(const float* x, long long n, const float* part, int nparts,
                                                       short* out) {
#pragma clang fp contract(off)
  __shared__ float scale_s;
  if (threadIdx.x == 0) {
    float m = 0.f;
    for (int p = 0; p < nparts; ++p) m = fmaxf(m, part[p]);
    const float amax = m / 0.99f;
    scale_s = amax > 1.0f ? 32768.0f / amax : 32768.0f;
  }
  __syncthreads();
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = (short)(int)(x[i] * scale_s);
}

inline unsigned blocks_for(long long n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

void launch_row_sqnorm(const float* x, float* out, long long rows, int cols, hipStream_t s) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(row_sqnorm_kernel, dim3(blocks_for(rows, 4)), dim3(256), 0, s, x, out, rows, cols);
  check_launch("row_sqnorm");
}

int knn_slices(int N) {
  // about 128 index rows per wave (a lane scans them one by one), at most
  // 256 slices, so F / 64 x slices waves fill the GPU for the usual few
  // hundred query frames; the merge reads slices x 8 candidates per query
  int S = (N + 127) / 128;
  return S < 1 ? 1 : (S > 256 ? 256 : S);
}

void launch_knn(const float* dot, long long ldd, const float* q2, const float* d2, int F, int N, int k,
                float* part_s, int* part_i, float* scores, long long* inds, hipStream_t s) {
  RVC_CHECK(k >= 1 && k <= kTopK, "knn: k must be in [1, 8]");
  if (F <= 0) return;
  const int S = knn_slices(N);
  const int per = (N + S - 1) / S;
  hipLaunchKernelGGL(knn_partial_kernel, dim3(blocks_for(F, 64), S), dim3(64), 0, s, dot, ldd, q2, d2, F, N, per,
                     part_s, part_i);
  check_launch("knn_partial");
  hipLaunchKernelGGL(knn_merge_kernel, dim3(blocks_for(F, 4)), dim3(256), 0, s, part_s, part_i, F, S, k, scores,
                     inds);
  check_launch("knn_merge");
}

size_t knn_part_entries(int F, int N) { return (size_t)knn_slices(N) * (size_t)(F > 0 ? F : 1) * kTopK; }

void launch_retrieval_blend(const float* scores, const long long* inds, const float* vecs, const float* feats,
                            float* out, int F, int D, int N, int k, float rate, float omr, hipStream_t s) {
  const long long n = (long long)F * D;
  if (n <= 0) return;
  hipLaunchKernelGGL(retrieval_blend_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, scores, inds, vecs, feats, out,
                     F, D, N, k, rate, omr);
  check_launch("retrieval_blend");
}

void launch_interp2_protect(const float* x, const float* x0, const float* pitchf, float protect, float* out, int F,
                            int D, hipStream_t s) {
  const long long n = 2LL * F * D;
  if (n <= 0) return;
  hipLaunchKernelGGL(interp2_protect_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, x, x0, pitchf, protect, out, F,
                     D);
  check_launch("interp2_protect");
}

void launch_rms_frames(const float* x, long long n, int hop, float* out, int frames, hipStream_t s) {
  if (frames <= 0) return;
  hipLaunchKernelGGL(rms_frames_kernel, dim3(frames), dim3(256), 0, s, x, n, hop, out);
  check_launch("rms_frames");
}

void launch_rms_mix(const float* data2, long long n2, const float* r1, int L1, const float* r2, int L2, float e1,
                    float e2, float* out, hipStream_t s) {
  if (n2 <= 0) return;
  hipLaunchKernelGGL(rms_mix_kernel, dim3(blocks_for(n2, 256)), dim3(256), 0, s, data2, n2, r1, L1, r2, L2, e1, e2,
                     out);
  check_launch("rms_mix");
}

int absmax_parts(long long n) {
  const long long b = (n + 255) / 256;
  return (int)(b < 1 ? 1 : (b > 1024 ? 1024 : b));
}

void launch_to_int16(const float* x, long long n, float* part, short* out, hipStream_t s) {
  if (n <= 0) return;
  const int parts = absmax_parts(n);
  hipLaunchKernelGGL(absmax_kernel, dim3(parts), dim3(256), 0, s, x, n, part);
  check_launch("absmax");
  hipLaunchKernelGGL(to_int16_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, x, n, part, parts, out);
  check_launch("to_int16");
}

}  // namespace rvc
