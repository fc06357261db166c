// Bandwidth-bound kernels: elementwise ops of the op-level ABI
// (runtime/vulkan_ops.py op set: leaky_relu, relu, copy, add/mul(_inplace),
// embedding, transpose), the NSF sine source, and the small glue kernels of
// the synthesis session (pitch-embedding combine, z_p sampling, WaveNet
// gate/update, flow channel flip, cond GEMV).
#include "internal.h"

// Keep numpy's rounding sequence for the elementwise formulas (no fused
// multiply-add contraction of a*b + c).
#pragma clang fp contract(off)

namespace rvc {
namespace {

unsigned grid1d(long long n) { return (unsigned)((n + 255) / 256); }

#define GRID_STRIDE(i, n) \
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < (n); i += (long long)gridDim.x * blockDim.x)

unsigned capped_grid(long long n) {
  long long g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  return (unsigned)(g < 1 ? 1 : g);
}

__global__ void leaky_kernel(float* a, long long n, float slope) {
  GRID_STRIDE(i, n) {
    const float v = a[i];
    a[i] = v >= 0.f ? v : slope * v;
  }
}
__global__ void relu_kernel(float* a, long long n) {
  GRID_STRIDE(i, n) a[i] = fmaxf(a[i], 0.f);
}
__global__ void copy_kernel(float* d, const float* s, long long n) {
  GRID_STRIDE(i, n) d[i] = s[i];
}
__global__ void add_inplace_kernel(float* a, const float* b, long long n) {
  GRID_STRIDE(i, n) a[i] = a[i] + b[i];
}
__global__ void mul_inplace_kernel(float* a, const float* b, long long n) {
  GRID_STRIDE(i, n) a[i] = a[i] * b[i];
}
__global__ void add_kernel(float* c, const float* a, const float* b, long long n) {
  GRID_STRIDE(i, n) c[i] = a[i] + b[i];
}
__global__ void mul_kernel(float* c, const float* a, const float* b, long long n) {
  GRID_STRIDE(i, n) c[i] = a[i] * b[i];
}
__global__ void fill_kernel(float* a, long long n, float v) {
  GRID_STRIDE(i, n) a[i] = v;
}
// out = a + gelu(p)   (HuBERT encoder entry: h + pos_conv_embed(h),
// runtime/models/hubert.py:855-857, :940)
__global__ void add_gelu_kernel(float* o, const float* a, const float* p, long long n) {
  GRID_STRIDE(i, n) o[i] = a[i] + gelu_as(p[i]);
}
// in-place GELU (erf form, the A&S 7.1.26 erf of gelu_as)
__global__ void gelu_kernel(float* a, long long n) {
  GRID_STRIDE(i, n) a[i] = gelu_as(a[i]);
}
// out[i] = a[i] + bias[i % cols]  (row-major [rows][cols] plus a per-column bias)
__global__ void bias_add_kernel(float* o, const float* a, const float* bias, long long n, long long cols) {
  GRID_STRIDE(i, n) o[i] = a[i] + bias[i % cols];
}
__global__ void avg3_kernel(float* o, const float* a, const float* b, const float* c, long long n) {
  GRID_STRIDE(i, n) o[i] = div3_rn((a[i] + b[i]) + c[i]);
}

// ids are validated by the host; the clamp only keeps a bad device-resident
// id from reading outside the table.
__global__ void embed_i32_kernel(const int* ids, const float* table, float* out, long long n, int rows,
                                 int dim) {
  GRID_STRIDE(e, n * dim) {
    const long long r = e / dim;
    const int c = (int)(e - r * dim);
    int id = ids[r];
    if (id < 0) id += rows;
    id = min(max(id, 0), rows - 1);
    out[e] = table[(long long)id * dim + c];
  }
}

// 32x32 tiled transpose through LDS (padded row to avoid bank conflicts).
__global__ __launch_bounds__(256) void transpose_kernel(const float* src, float* out, int C, int P,
                                                        float scale) {
  __shared__ float tile[32][33];
  const int b = blockIdx.z;
  const float* sb = src + (long long)b * C * P;
  float* ob = out + (long long)b * C * P;
  const int p0 = blockIdx.x * 32, c0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int r = ty; r < 32; r += 8) {
    const int c = c0 + r, p = p0 + tx;
    if (c < C && p < P) tile[r][tx] = sb[(long long)c * P + p];
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    const int p = p0 + r, c = c0 + tx;
    if (c < C && p < P) ob[(long long)p * C + c] = tile[tx][r] * scale;
  }
}

__global__ void flip_kernel(const float* src, float* dst, int C, long long L, long long n) {
  GRID_STRIDE(e, n) {
    const long long t = e % L;
    const long long bc = e / L;
    const int c = (int)(bc % C);
    const long long b = bc / C;
    dst[e] = src[(b * C + (C - 1 - c)) * L + t];
  }
}

// An id outside [-rows, rows) (numpy's take would raise) sets bit 0 of *err
// for the host to report; the read itself is clamped so it stays in bounds.
__global__ void embed_combine_kernel(const float* E, const long long* pitch, const float* table, float* x,
                                     int C, int P, int rows, float scale, float slope, long long n,
                                     unsigned* err) {
  GRID_STRIDE(e, n) {
    const int t = (int)(e % P);
    const long long bc = e / P;
    const int c = (int)(bc % C);
    const long long b = bc / C;
    long long id = pitch[b * P + t];
    if ((id < -rows || id >= rows) && err) atomicOr(err, 1u);
    if (id < 0) id += rows;
    id = id < 0 ? 0 : (id >= rows ? rows - 1 : id);
    float v = E[e] + table[id * C + c];
    v = v * scale;
    x[e] = v >= 0.f ? v : slope * v;
  }
}

__device__ __forceinline__ float sigmoid_ref(float x) {
  // both-branch stable form of runtime/nn.py:520-523
  if (x >= 0.f) return 1.0f / (1.0f + expf(-x));
  const float e = expf(x);
  return e / (1.0f + e);
}

__global__ void wn_gate_kernel(const float* XI, long long xib, const float* g, long long gb, float* acts,
                               int H, int L, long long n) {
  GRID_STRIDE(e, n) {
    const int t = (int)(e % L);
    const long long bc = e / L;
    const int c = (int)(bc % H);
    const long long b = bc / H;
    const float* xi = XI + b * xib;
    const float* gg = g + b * gb;
    const float a1 = xi[(long long)c * L + t] + gg[c];
    const float a2 = xi[(long long)(H + c) * L + t] + gg[H + c];
    acts[e] = tanhf(a1) * sigmoid_ref(a2);
  }
}

// op 18 of the record/commit API (engine/shaders/gating.comp semantics)
__global__ void gating_kernel(const float* a, const float* g, float* c, long long n, int lg, int h,
                              long long off) {
  GRID_STRIDE(i, n) {
    const long long L = n / h;
    const long long hlg = (long long)h * lg;
    const long long bi = (lg == 1) ? off + i / L : off + (i / L) * lg + (i % L);
    c[i] = tanhf(a[i] + g[bi]) * sigmoid_ref(a[i + n] + g[bi + hlg]);
  }
}

__global__ void zp_kernel(const float* st, const float* nz, float* z, int H, int L, float k, long long n) {
  GRID_STRIDE(e, n) {
    const int t = (int)(e % L);
    const long long bc = e / L;
    const int c = (int)(bc % H);
    const long long b = bc / H;
    const float* sb = st + b * 2 * H * (long long)L;
    const float m = sb[(long long)c * L + t];
    const float lg = sb[(long long)(H + c) * L + t];
    z[e] = m + expf(lg) * nz[e] * k;
  }
}

__global__ void wn_update_kernel(float* h, float* skip, const float* rs, int H, int L, int first,
                                 int last, long long n) {
  GRID_STRIDE(e, n) {
    const int t = (int)(e % L);
    const long long bc = e / L;
    const int c = (int)(bc % H);
    const long long b = bc / H;
    if (last) {
      const float v = rs[(b * H + c) * (long long)L + t];
      skip[e] = first ? v : skip[e] + v;
    } else {
      const float* rb = rs + b * 2 * H * (long long)L;
      h[e] = h[e] + rb[(long long)c * L + t];
      const float v = rb[(long long)(H + c) * L + t];
      skip[e] = first ? v : skip[e] + v;
    }
  }
}

__global__ void sub_strided_kernel(float* x1, long long x1b, const float* m, long long mb, int C, int L,
                                   long long n) {
  GRID_STRIDE(e, n) {
    const long long ct = e % ((long long)C * L);
    const long long b = e / ((long long)C * L);
    float* p = x1 + b * x1b + ct;
    *p = *p - m[b * mb + ct];
  }
}

// out-of-range ids set bit 1 of *err (reads clamped, as above)
__global__ void gather_rows_i64_kernel(const long long* ids, const float* table, float* out, int rows,
                                       int dim, long long n, unsigned* err) {
  GRID_STRIDE(e, n) {
    const long long b = e / dim;
    const int c = (int)(e - b * dim);
    long long id = ids[b];
    if ((id < -rows || id >= rows) && err) atomicOr(err, 2u);
    if (id < 0) id += rows;
    id = id < 0 ? 0 : (id >= rows ? rows - 1 : id);
    out[e] = table[id * dim + c];
  }
}

// One wave per output row: lanes stride the row (coalesced), then a
// butterfly reduction.
__global__ __launch_bounds__(256) void gemv_kernel(const float* W, const float* bias, const float* g, long long gb,
                                                   float* out, long long ob, int C_out, int C_in, long long n) {
  const long long e = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (e >= n) return;
  const int co = (int)(e % C_out);
  const long long b = e / C_out;
  const float* gg = g + b * gb;
  const float* wr = W + (long long)co * C_in;
  float acc = 0.f;
  for (int ci = lane; ci < C_in; ci += 64) acc += wr[ci] * gg[ci];
  for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
  if (lane == 0) out[b * ob + co] = acc + bias[co];
}

// ---- NSF sine source (runtime/models/vits.py:1468-1501) ----
// Per-frame phase of the NSF source.  rad_acc[p] = fmod(sum_{q<=p} r2[q], 1)
// with r2[q] = fmod(f0[q]/sr*upp + 0.5, 1) - 0.5, the sum taken sequentially
// in float32 (numpy's cumsum order, vits.py:1482-1488), is the reference's
// _phase_offsets (:2404-2414).  out[p + shift] = rad_acc[p]: shift 0 writes
// rad_acc itself; shift 1 writes the offset each frame's phase adds (0 for
// frame 0, rad_acc[p-1] after it), the form the har kernel reads.
//
// Any P: the frames go through LDS in blocks of kPhaseBlock.  For each block
// the workgroup forms r2 in parallel, one thread continues the running sum
// over the block (the same sequential additions, carried from the previous
// block in a register), and the fmod of every prefix is taken and stored in
// parallel.  The serial thread reads its operands 16 at a time as float4s
// and writes the prefixes back the same way, so the dependent chain is the
// float additions themselves, not one LDS round trip per frame.
constexpr int kPhaseBlock = 4096;

__global__ __launch_bounds__(256) void sine_phase_kernel(const float* f0, float* out, int P, int upp,
                                                         float sr, int shift) {
  __shared__ float4 r4[kPhaseBlock / 4];
  float* r2 = reinterpret_cast<float*>(r4);
  const int b = blockIdx.x;
  const float* fb = f0 + (long long)b * P;
  float* ob = out + (long long)b * P;
  float c = 0.f;  // running sum (thread 0)
  for (int p0 = 0; p0 < P; p0 += kPhaseBlock) {
    const int n = min(kPhaseBlock, P - p0);
    for (int p = threadIdx.x; p < kPhaseBlock; p += blockDim.x) {
      float v = 0.f;  // the block's tail past P stays 0 and is never stored
      if (p < n) {
        const float rl = (fb[p0 + p] / sr) * (float)upp;
        v = fmodf(rl + 0.5f, 1.0f) - 0.5f;
      }
      r2[p] = v;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      // frame 0 starts the sum with r2[0] itself, as numpy's cumsum does
      for (int q = 0; q < (n + 15) / 16; ++q) {
        float4 a = r4[4 * q], bq = r4[4 * q + 1], cq = r4[4 * q + 2], dq = r4[4 * q + 3];
        if (p0 == 0 && q == 0) {
          c = a.x;
        } else {
          c = c + a.x;
        }
        a.x = c;
        c = c + a.y; a.y = c;
        c = c + a.z; a.z = c;
        c = c + a.w; a.w = c;
        c = c + bq.x; bq.x = c;
        c = c + bq.y; bq.y = c;
        c = c + bq.z; bq.z = c;
        c = c + bq.w; bq.w = c;
        c = c + cq.x; cq.x = c;
        c = c + cq.y; cq.y = c;
        c = c + cq.z; cq.z = c;
        c = c + cq.w; cq.w = c;
        c = c + dq.x; dq.x = c;
        c = c + dq.y; dq.y = c;
        c = c + dq.z; dq.z = c;
        c = c + dq.w; dq.w = c;
        r4[4 * q] = a; r4[4 * q + 1] = bq; r4[4 * q + 2] = cq; r4[4 * q + 3] = dq;
      }
      // c carries into the next block; only the last block can be partial,
      // so the padding zeros it adds are never carried
    }
    __syncthreads();
    for (int p = threadIdx.x; p < n; p += blockDim.x)
      if (p0 + p + shift < P) ob[p0 + p + shift] = fmodf(r2[p], 1.0f);
    __syncthreads();  // r2 is refilled by the next block
  }
  if (shift && threadIdx.x == 0) ob[0] = 0.f;
}

// har[b][p*upp+u] = tanh(w * (0.1*sin(2pi*rad)*uv + amp*ns) + b) with
// rad = (f0[p]/sr)*(u+1) + off[p]   (float32, numpy's evaluation order).
// off[p] is the frame's whole phase offset: rad_acc[p-1] (0 at p = 0) for a
// full synthesis -- adding 0.0 to frame 0 leaves it bit-identical -- or the
// caller's seg_offsets for a segment (runtime/models/vits.py:1484-1491).
__global__ void sine_har_kernel(const float* f0, const float* ns, const float* off, float* har, int P,
                                int upp, float sr, float w_lin, float b_lin, long long n) {
  const float two_pi = 6.2831855f;  // float32(2*pi), as numpy rounds the python scalar
  GRID_STRIDE(e, n) {
    const long long per = (long long)P * upp;
    const long long b = e / per;
    const long long j = e - b * per;
    const int p = (int)(j / upp);
    const int u = (int)(j - (long long)p * upp);
    const float f = f0[b * P + p];
    const float rad = (f / sr) * (float)(u + 1) + off[b * P + p];
    const float sine = sinf(two_pi * rad) * 0.1f;
    const float uv = f > 0.f ? 1.f : 0.f;
    const float amp = uv * 0.003f + ((1.f - uv) * 0.1f) / 3.f;
    const float v = sine * uv + amp * ns[e];
    har[e] = tanhf(v * w_lin + b_lin);
  }
}

}  // namespace

void launch_leaky(float* a, long long n, float slope, hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(leaky_kernel, dim3(capped_grid(n)), dim3(256), 0, s, a, n, slope);
  check_launch("leaky_relu");
}
void launch_relu(float* a, long long n, hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(relu_kernel, dim3(capped_grid(n)), dim3(256), 0, s, a, n);
  check_launch("relu");
}
void launch_copy(float* d, const float* src, long long n, hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(copy_kernel, dim3(capped_grid(n)), dim3(256), 0, s, d, src, n);
  check_launch("copy");
}
void launch_add_inplace(float* a, const float* b, long long n, hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(add_inplace_kernel, dim3(capped_grid(n)), dim3(256), 0, s, a, b, n);
  check_launch("add_inplace");
}
void launch_mul_inplace(float* a, const float* b, long long n, hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(mul_inplace_kernel, dim3(capped_grid(n)), dim3(256), 0, s, a, b, n);
  check_launch("mul_inplace");
}
void launch_add(float* c, const float* a, const float* b, long long n, hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(add_kernel, dim3(capped_grid(n)), dim3(256), 0, s, c, a, b, n);
  check_launch("add");
}
void launch_mul(float* c, const float* a, const float* b, long long n, hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(mul_kernel, dim3(capped_grid(n)), dim3(256), 0, s, c, a, b, n);
  check_launch("mul");
}
void launch_fill(float* a, long long n, float v, hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(fill_kernel, dim3(capped_grid(n)), dim3(256), 0, s, a, n, v);
  check_launch("fill");
}
void launch_add_gelu(float* out, const float* a, const float* p, long long n, hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(add_gelu_kernel, dim3(capped_grid(n)), dim3(256), 0, s, out, a, p, n);
  check_launch("add_gelu");
}
void launch_gelu(float* a, long long n, hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(gelu_kernel, dim3(capped_grid(n)), dim3(256), 0, s, a, n);
  check_launch("gelu");
}
void launch_bias_add(float* out, const float* a, const float* bias, long long n, long long cols, hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(bias_add_kernel, dim3(capped_grid(n)), dim3(256), 0, s, out, a, bias, n, cols);
  check_launch("bias_add");
}

void launch_avg3(float* out, const float* a, const float* b, const float* c, long long n, hipStream_t s) {
  if (n <= 0) return;
  launch_timed(avg3_kernel, dim3(capped_grid(n)), dim3(256), 0, s, out, a, b, c, n);
  check_launch("avg3");
}
void launch_embed_i32(const int* ids, const float* table, float* out, long long n, int rows, int dim,
                      hipStream_t s) {
  if (n <= 0 || dim <= 0) return;
  hipLaunchKernelGGL(embed_i32_kernel, dim3(capped_grid(n * dim)), dim3(256), 0, s, ids, table, out, n,
                     rows, dim);
  check_launch("embed");
}
void launch_transpose(const float* src, float* out, int B, int C, int P, float scale, hipStream_t s) {
  if ((long long)B * C * P == 0) return;
  dim3 grid((P + 31) / 32, (C + 31) / 32, B);
  hipLaunchKernelGGL(transpose_kernel, grid, dim3(256), 0, s, src, out, C, P, scale);
  check_launch("transpose");
}
void launch_flip_channels(const float* src, float* dst, int B, int C, int L, hipStream_t s) {
  const long long n = (long long)B * C * L;
  if (n <= 0) return;
  hipLaunchKernelGGL(flip_kernel, dim3(capped_grid(n)), dim3(256), 0, s, src, dst, C, (long long)L, n);
  check_launch("flip_channels");
}
void launch_embed_combine(const float* E, const long long* pitch, const float* table, int rows, float* x,
                          int B, int C, int P, float scale, float slope, unsigned* err, hipStream_t s) {
  const long long n = (long long)B * C * P;
  if (n <= 0) return;
  hipLaunchKernelGGL(embed_combine_kernel, dim3(capped_grid(n)), dim3(256), 0, s, E, pitch, table, x, C,
                     P, rows, scale, slope, n, err);
  check_launch("embed_combine");
}
void launch_wn_gate(const float* XI, long long xib, const float* g, long long gb, float* acts, int B,
                    int H, int L, hipStream_t s) {
  const long long n = (long long)B * H * L;
  if (n <= 0) return;
  hipLaunchKernelGGL(wn_gate_kernel, dim3(capped_grid(n)), dim3(256), 0, s, XI, xib, g, gb, acts, H, L, n);
  check_launch("wn_gate");
}
void launch_gating(const float* a, const float* g, float* c, long long n, int lg, int h, long long off,
                   hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(gating_kernel, dim3(capped_grid(n)), dim3(256), 0, s, a, g, c, n, lg, h, off);
  check_launch("gating");
}
void launch_zp(const float* st, const float* nz, float* z, int B, int H, int L, float k, hipStream_t s) {
  const long long n = (long long)B * H * L;
  if (n <= 0) return;
  hipLaunchKernelGGL(zp_kernel, dim3(capped_grid(n)), dim3(256), 0, s, st, nz, z, H, L, k, n);
  check_launch("zp");
}
void launch_wn_update(float* h, float* skip, const float* rs, int B, int H, int L, int first, int last,
                      hipStream_t s) {
  const long long n = (long long)B * H * L;
  if (n <= 0) return;
  hipLaunchKernelGGL(wn_update_kernel, dim3(capped_grid(n)), dim3(256), 0, s, h, skip, rs, H, L, first,
                     last, n);
  check_launch("wn_update");
}
void launch_sub_inplace_strided(float* x1, long long x1b, const float* m, long long mb, int B, int C,
                                int L, hipStream_t s) {
  const long long n = (long long)B * C * L;
  if (n <= 0) return;
  hipLaunchKernelGGL(sub_strided_kernel, dim3(capped_grid(n)), dim3(256), 0, s, x1, x1b, m, mb, C, L, n);
  check_launch("sub_inplace");
}
void launch_gather_rows_i64(const long long* ids, const float* table, float* out, int B, int rows, int dim,
                            unsigned* err, hipStream_t s) {
  const long long n = (long long)B * dim;
  if (n <= 0) return;
  hipLaunchKernelGGL(gather_rows_i64_kernel, dim3(capped_grid(n)), dim3(256), 0, s, ids, table, out, rows, dim,
                     n, err);
  check_launch("gather_rows");
}
void launch_gemv(const float* W, const float* bias, const float* g, long long gb, float* out, long long ob,
                 int B, int C_out, int C_in, hipStream_t s) {
  const long long n = (long long)B * C_out;
  if (n <= 0) return;
  hipLaunchKernelGGL(gemv_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s, W, bias, g, gb, out, ob, C_out,
                     C_in, n);
  check_launch("gemv");
}
void launch_sine_phase(const float* f0, float* out, int B, int P, int upp, float sr, int shift, hipStream_t s) {
  if ((long long)B * P == 0) return;
  hipLaunchKernelGGL(sine_phase_kernel, dim3(B), dim3(256), 0, s, f0, out, P, upp, sr, shift);
  check_launch("sine_phase");
}
void launch_sine_source(const float* f0, const float* ns, float* har, float* off, const float* seg_off, int B, int P,
                        int upp, float sr, float w_lin, float b_lin, hipStream_t s) {
  if ((long long)B * P == 0) return;
  if (!seg_off) launch_sine_phase(f0, off, B, P, upp, sr, 1, s);
  const long long n = (long long)B * P * upp;
  hipLaunchKernelGGL(sine_har_kernel, dim3(capped_grid(n)), dim3(256), 0, s, f0, ns, seg_off ? seg_off : off, har, P,
                     upp, sr, w_lin, b_lin, n);
  check_launch("sine_har");
}

}  // namespace rvc
