// The end of one reverse flow and the start of the next as one kernel
// (runtime/models/vits.py:1086-1145, 1255-1268):
//
//   skip'  = skip + (W_rs acts + b_rs)        the WaveNet's last res/skip layer
//                                             (skip rows only)
//   x1'    = x1 - (W_post skip' + b_post)     post conv, mean-only coupling
//   h_next = W_pre' x1' + b_pre'              the next flow's pre conv
//
// The next flow's pre conv reads exactly the half this flow updates (the
// flips alternate which physical half of X is x0; the weights are arranged
// for it at load), so one workgroup that owns BN = 16 frames and all C
// channels can run the three 1x1 convolutions back to back with the
// intermediate tiles in LDS.  It replaces three launches (the last res/skip
// conv, post, the next pre) and skip' never goes to memory.  Wave w computes
// rows [16w, 16w + 16) of each product over its whole reduction with
// v_mfma_f32_16x16x4_f32 (lane l: A row l % 16, k l / 16; accumulator g:
// row 4 (l / 16) + g, column l % 16); its weights of all three products are
// loaded into registers at the start, with the epilogue operands, so the
// kernel waits on global memory once.
#include "internal.h"

namespace rvc {

typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int BN = 16;  // frames per workgroup

template <int RT>
__global__ __launch_bounds__(64 * RT) void flow_tail_kernel(FlowTailArgs a) {
  constexpr int C = 16 * RT, HALF = 8 * RT, NT = 64 * RT;
  constexpr int NPOST = RT / 2;  // waves holding the post conv's HALF rows
  __shared__ float xs[C * BN];     // acts tile [C][BN]
  __shared__ float ys[C * BN];     // skip' tile
  __shared__ float zs[HALF * BN];  // x1' tile
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int kq = lane >> 4;
  const int l16 = lane & 15;
  const int b = blockIdx.y;
  const int t0 = blockIdx.x * BN;
  const int P = a.P;
  const int co0 = 16 * wave;
  const bool lcol = t0 + l16 < P;  // this lane's accumulator column
  const unsigned cp = 4u * (unsigned)P;  // bytes per channel row

  // ---- every global operand in flight at once ----
  // weights: A[row l16][k 4s + kq] = W[co0 + l16][4s + kq], in lane order
  // (pack_mfma_lanes): step group j is one float4 per lane, the wave's 64 of
  // them contiguous
  float wrv[C / 4], wpv[C / 4], wqv[HALF / 4];
  auto load_rows = [&](const float* w, int rows, int K, bool on, float* dst) {
    const __amdgpu_buffer_rsrc_t rs = uniform_rsrc(w, 4u * (unsigned)(rows * K));
    const unsigned o = on ? 16u * (unsigned)(wave * (K / 16) * 64 + lane) : kBufOut;
#pragma unroll
    for (int s = 0; s < K / 16; ++s) {
      const float4 v = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, o, 1024u * s, 0));
      dst[4 * s] = v.x;
      dst[4 * s + 1] = v.y;
      dst[4 * s + 2] = v.z;
      dst[4 * s + 3] = v.w;
    }
  };
  load_rows(a.w_rs, C, C, true, wrv);
  load_rows(a.w_post, HALF, C, wave < NPOST, wpv);
  load_rows(a.w_pre ? a.w_pre : a.w_post, C, HALF, a.w_pre != nullptr, wqv);
  // epilogue operands: rows co0 + 4 kq + g, column t0 + l16
  const unsigned eo = lcol ? 4u * (unsigned)((co0 + 4 * kq) * P + t0 + l16) : kBufOut;
  const __amdgpu_buffer_rsrc_t srs = uniform_rsrc(a.skip + (long long)b * C * P, cp * C);
  const __amdgpu_buffer_rsrc_t xrs = uniform_rsrc(a.x1 + (long long)b * a.xb, cp * HALF);
  float sv[4], xv[4], brs[4], bpo[4], bpr[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int co = co0 + 4 * kq + g;
    sv[g] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(srs, eo, g * cp, 0));
    xv[g] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xrs, wave < NPOST ? eo : kBufOut, g * cp, 0));
    brs[g] = a.b_rs[co];
    bpo[g] = wave < NPOST ? a.b_post[co] : 0.f;
    bpr[g] = a.w_pre ? a.b_pre[co] : 0.f;
  }
  // the acts tile: thread (row tid / BN + (NT / BN) j, column tid % BN)
  {
    const int col = tid % BN;
    const __amdgpu_buffer_rsrc_t ars = uniform_rsrc(a.acts + (long long)b * C * P, cp * C);
    const bool ok = t0 + col < P;
#pragma unroll
    for (int j = 0; j < C * BN / NT; ++j) {
      const int r = tid / BN + (NT / BN) * j;
      xs[tid + NT * j] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(ars, ok ? 4u * (unsigned)(r * P + t0 + col) : kBufOut, 0, 0));
    }
  }
  __syncthreads();

  // ---- skip' = skip + (W_rs acts + b_rs) ----
  {
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    const float* bl = xs + kq * BN + l16;
#pragma unroll
    for (int s = 0; s < C / 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wrv[s], bl[4 * s * BN], acc, 0, 0, 0);
#pragma unroll
    for (int g = 0; g < 4; ++g) ys[(co0 + 4 * kq + g) * BN + l16] = sv[g] + (acc[g] + brs[g]);
  }
  __syncthreads();

  // ---- x1' = x1 - (W_post skip' + b_post) ----
  if (wave < NPOST) {
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    const float* bl = ys + kq * BN + l16;
#pragma unroll
    for (int s = 0; s < C / 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wpv[s], bl[4 * s * BN], acc, 0, 0, 0);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float v = xv[g] - (acc[g] + bpo[g]);
      zs[(co0 + 4 * kq + g) * BN + l16] = v;
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), xrs, eo, g * cp, 0);
    }
  }
  if (!a.w_pre) return;  // uniform: no barrier follows
  __syncthreads();

  // ---- h_next = W_pre' x1' + b_pre' ----
  {
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    const float* bl = zs + kq * BN + l16;
#pragma unroll
    for (int s = 0; s < HALF / 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wqv[s], bl[4 * s * BN], acc, 0, 0, 0);
    const __amdgpu_buffer_rsrc_t hrs = uniform_rsrc(a.h + (long long)b * C * P, cp * C);
#pragma unroll
    for (int g = 0; g < 4; ++g)
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, acc[g] + bpr[g]), hrs, eo, g * cp, 0);
  }
}

}  // namespace

bool flow_tail_supported(int C, int half) { return (C == 128 || C == 192) && 2 * half == C; }

void launch_flow_tail(const FlowTailArgs& a, int C, int B, hipStream_t s) {
  RVC_CHECK(flow_tail_supported(C, C / 2), "flow_tail: unsupported channel count");
  RVC_CHECK(a.P >= 1 && B >= 1 && a.xb >= (long long)(C / 2) * a.P, "flow_tail: invalid shape");
  RVC_CHECK(a.w_rs && a.w_post && (!a.w_pre || (a.h && a.b_pre)), "flow_tail: missing weights");
  // 32-bit byte offsets within one batch item's [C][P] tensors
  RVC_CHECK(4.0 * C * a.P < 2147483648.0, "flow_tail: sequence too long for 32-bit offsets");
  const dim3 grid((unsigned)((a.P + BN - 1) / BN), (unsigned)B);
  if (C == 128)
    hipLaunchKernelGGL(flow_tail_kernel<8>, grid, dim3(64 * 8), 0, s, a);
  else
    hipLaunchKernelGGL(flow_tail_kernel<12>, grid, dim3(64 * 12), 0, s, a);
  check_launch("flow_tail");
}

}  // namespace rvc
