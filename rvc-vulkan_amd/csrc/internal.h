// Internal declarations shared by the HIP kernels, the engine and the C ABI.
//
// Layout convention inside the engine: every activation tensor is stored
// channel-major per batch item, [B][C][L] with time contiguous (the PyTorch
// NCT layout the reference uses for conv1d, runtime/nn.py:8-12).  Strides
// are passed explicitly so kernels can read channel slices in place.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

namespace rvc {

// ---------------------------------------------------------------- errors
struct Error : std::runtime_error {
  explicit Error(const std::string& m) : std::runtime_error(m) {}
};

void set_last_error(const std::string& msg);

#define RVC_HIP(expr)                                                        \
  do {                                                                       \
    hipError_t _e = (expr);                                                  \
    if (_e != hipSuccess)                                                    \
      throw ::rvc::Error(std::string(#expr) + ": " + hipGetErrorString(_e)); \
  } while (0)

#define RVC_CHECK(cond, msg)                 \
  do {                                       \
    if (!(cond)) throw ::rvc::Error(msg);    \
  } while (0)

void check_launch(const char* what);

// Kernel-end events without a marker packet.  An event recorded between two
// kernels is a marker the command processor runs between them, idling the
// GPU for a few microseconds; a stop event attached to the kernel's own
// dispatch (hipExtLaunchKernelGGL) costs nothing.  While a session times a
// launch, stop_hook().ev is the end event of its timing span: the launch
// sites that end their call's work with one kernel (the persistent, small
// and 1x1 conv kernels, the ConvTranspose, conv_post, stage-0 noise conv and
// ResBlock-average kernels) launch through launch_timed(),
// which attaches it and counts the launch in `used`; the session records
// the event itself when no launch did.
struct StopHook {
  hipEvent_t ev = nullptr;
  int used = 0;
};
StopHook& stop_hook();  // this thread's
template <typename F, typename... Args>
inline void launch_timed(F kernel, dim3 grid, dim3 block, size_t lds, hipStream_t s, Args... args) {
  StopHook& h = stop_hook();
  if (h.ev) {
    hipExtLaunchKernelGGL(kernel, grid, block, (std::uint32_t)lds, s, nullptr, h.ev, 0u, args...);
    ++h.used;
  } else {
    hipLaunchKernelGGL(kernel, grid, block, lds, s, args...);
  }
}

// ---------------------------------------------------------------- conv args
// Activation applied while loading an input tile (prologue) or before the
// combine step of the epilogue.
enum Act : int { ACT_NONE = 0, ACT_LEAKY = 1, ACT_TANH = 2, ACT_RELU = 3, ACT_GELU = 4, ACT_SIGMOID = 5 };

// A raw buffer resource (32-bit offsets, out-of-range reads give 0 and
// out-of-range writes are dropped) from values the whole wave shares.
// readfirstlane keeps the descriptor in scalar registers even where the
// compiler placed one of its inputs in a vector register (a descriptor in
// vector registers turns every load through it into a waterfall loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const void* base, unsigned range) {
  const unsigned long long v = reinterpret_cast<unsigned long long>(base);
  const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v);
  const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
  void* p = reinterpret_cast<void*>(((unsigned long long)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(p, (short)0, (int)__builtin_amdgcn_readfirstlane(range), 0x00020000);
}
// the offset a masked lane passes: above every range these kernels build
constexpr unsigned kBufOut = 0x80000000u;
// Direct-to-LDS buffer loads: lane i of the wave writes its 4 (16) bytes at
// lds + 4 i (16 i), an out-of-range lane writes 0; `lds` is the same for the
// whole wave.  The wave waits for them with s_waitcnt vmcnt before a barrier.
__device__ __forceinline__ void buffer_load_lds_b32(__amdgpu_buffer_rsrc_t r, float* lds, unsigned off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 4, off, 0, 0, 0);
}
__device__ __forceinline__ void buffer_load_lds_b128(__amdgpu_buffer_rsrc_t r, float4* lds, unsigned off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, off, 0, 0, 0);
}

// x / 3 rounded to nearest (the decoder's ResBlock average) in five VALU
// operations instead of the full division sequence: q0 = RN(x * r) with
// r = RN(1/3), the remainder x - 3 q0 by one fused multiply-add, and
// q = RN(q0 + remainder * r).  q is bit-identical to the IEEE quotient for
// every finite non-zero float (all 2^32 bit patterns checked on the host);
// zeros and infinities, where the remainder is 0 or NaN, take q0, which is
// then the exact quotient with its sign.
__device__ __forceinline__ float div3_rn(float x) {
  constexpr float r = 0x1.555556p-2f;
  const float q0 = __fmul_rn(x, r);
  const float q = __builtin_fmaf(__builtin_fmaf(-q0, 3.0f, x), r, q0);
  return (q0 == 0.f || __builtin_isinf(q0)) ? q0 : q;
}

// logistic function in the two-branch form of runtime/nn.py:520-523
__device__ inline float sigmoid_as(float x) {
  if (x >= 0.f) return 1.0f / (1.0f + expf(-x));
  const float e = expf(x);
  return e / (1.0f + e);
}

// GELU with erf by Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7), the
// formula and float32 operation order of the reference's numpy gelu_erf
// (runtime/models/hubert.py:194-202, :222-241): u = x / sqrt 2,
// erf(u) = sign(u) (1 - poly(t) t exp(-u^2)) with t = 1 / (1 + p |u|).
__device__ inline float gelu_as(float x) {
#pragma clang fp contract(off)
  const float u = x * 0.7071067811865476f;
  const float au = fabsf(u);
  const float t = 1.0f / (1.0f + 0.3275911f * au);
  const float poly = ((((1.061405429f * t + -1.453152027f) * t) + 1.421413741f) * t + -0.284496736f) * t +
                     0.254829592f;
  const float y = 1.0f - poly * t * expf(-au * au);
  const float e = u > 0.f ? y : (u < 0.f ? -y : 0.f);
  return 0.5f * x * (1.0f + e);
}

// How the epilogue value v = act((acc + bias [+ bias2]) [+ res]) lands in out.
enum Combine : int {
  COMB_STORE = 0,    // out = v
  COMB_ADD = 1,      // out = out + v
  COMB_ADD_DIV = 2,  // out = (out + v) / div
  COMB_SUB = 3,      // out = out - v (the small-conv kernels only: conv1d_mfma_small_path)
};

// MFMA fast path bounds: taps per conv and the input halo (K-1)*dil.
constexpr int kConvTapsMax = 11;
constexpr int kConvHaloMax = 64;
constexpr int kMaxConvGroups = 16;

// One convolution of a grouped MFMA launch (fields that differ per group).
struct ConvGroup {
  const float* x;     // input [B][C_in (stride xc)][L_in]
  const float* w;     // packed weights [K][C_in][w_ld], 16-byte aligned
  const float* bias;  // [C_out] or null
  const float* res;   // residual, indexed like out, or null
  float* out;
  int K, dil;
  int in_off;         // input index of output i, tap k: i * in_step + in_off + k * dil
  int in_step;        // input stride (0 or 1: stride 1; 2 supported)
  int out_step;       // output element index = i * out_step + out_off
  int out_off;
  int n_out;
  int combine;
  const uint16_t* w16;  // bf16 launches: weights [K][C_out][w16_ld] in bf16, 16-byte aligned
  int tiles;          // output tiles per workgroup (set by the launcher)
};

// A launch of up to kMaxConvGroups convolutions with the same channel
// counts, strides and activations (grid z = group * B + batch).
struct ConvLaunch {
  ConvGroup g[kMaxConvGroups];
  int n_groups;
  long long xb, xc;   // batch / channel stride of x
  long long ob, oc;   // of out
  long long rb, rc;   // of res
  const float* bias2; // second per-channel addend [B][C_out] or null
  long long bias2b;
  int C_in, C_out, w_ld, L_in, B;
  int w16_ld;  // bf16 weight row length (C_in rounded up to 8, zero padded)
  int in_act;  float in_slope;
  int out_act; float out_slope;
  float div;
  // split-K over workgroups (single-group stride-1 launches): scratch for the
  // partial sums, filled in by the launcher when part_floats suffices
  float* part;
  size_t part_floats;
  int ksplit, csplit;  // set by the launcher
  // the chunked 1x1 small-conv kernel's reduction split over sc_split
  // workgroups (set by the launcher; the partial tiles go to part, a reduce
  // launch forms the output)
  int sc_split;
  // what the split-K reduce (or the small-conv kernel) does with v = sum of
  // the splits + bias (the launch must take one of those paths:
  // conv1d_mfma_fuses_gate(a) for the gate):
  //   POST_WN_GATE   (C_out = 2H): out[c][t] = tanh(v_c + g[c]) * sig(v_{H+c} + g[H+c])
  //                  for c < H, out of row stride oc, g per batch item (stride post_gb)
  //   POST_WN_UPDATE (C_out = 2H, or H when post_last): h += v_c (c < H, not last),
  //                  skip = / += v of the skip channels (post_first: =)
  int post;
  const float* post_g; long long post_gb;
  float* post_h; float* post_skip;
  int post_H, post_first, post_last;
  // persistent launches: 9 zeroed counters (8 per-XCD item queues and a
  // finish count, reset by the launch's last workgroup) for dynamic item
  // scheduling; null: static round-robin.  One launch at a time per buffer.
  unsigned* queue;
  // LayerNorm of the input over its C_in channels, applied while it is
  // staged (the whole-reduction 1x1 kernel, single group, no input
  // activation): x' = (x - mean_t) * (1 / sqrt(var_t + ln_eps)) * ln_g[c] + ln_b[c]
  // per column t (two-pass, float64 sums, the formulas of the LayerNorm
  // kernels).  The workgroups of C_out tile 0 also store x' to ln_out
  // (batch / channel strides ln_ob / ln_oc), for the consumers of the
  // normalised tensor itself.  ln_g == null: no LayerNorm.
  const float* ln_g;
  const float* ln_b;
  float* ln_out;
  long long ln_ob, ln_oc;
  float ln_eps;
  // The same LayerNorm in the chunked small-conv kernel (1x1, single group),
  // whose chunks cannot hold a whole column: the statistics come from the
  // kernel that produced the input.  stat_out (producer, single group,
  // C_out % 32 == 0): per batch item, 32-row C_out tile and output column,
  // the float64 sum and sum of squares of the 32 values it stored, added in
  // row order, as double2 [B][C_out / 32][n_out].  ln_stat (consumer): its
  // input's statistics in that layout, ln_ntile = C_in / 32 tiles of L_in
  // columns, added in tile order: mean = S / C_in, var = (Q - S * mean) /
  // C_in, and x' = (x - mean) * (1 / sqrt(var + ln_eps)) while staging --
  // without the affine, which the caller folds into the weights (W diag(g))
  // and the bias (+ W b); ln_g / ln_b / ln_out unused.  res_stat: the
  // residual is such a raw tensor too (C_out channels, C_out / 32 tiles,
  // statistics over n_out columns), normalised with its affine res_g / res_b
  // (and ln_eps) before it is added, so no kernel stores the normalised
  // tensor.  The sums do not depend on the batch or the tile widths of any
  // launch.
  double* stat_out;
  const double* ln_stat;
  int ln_ntile;
  const double* res_stat;
  const float* res_g;
  const float* res_b;
};
enum Post : int { POST_NONE = 0, POST_WN_GATE = 1, POST_WN_UPDATE = 2 };

// MFMA implicit-GEMM conv1d (input stride 1 or 2, the same for every group
// of a launch), K <= kConvTapsMax and (K-1)*dil <= kConvHaloMax.
bool conv1d_mfma_supported(int K, int dil);
// launch_conv1d_mfma would run `a` (stride 1) on the chunked small-conv
// kernel as a 1x1 GEMM: the launches that can take ln_stat
bool conv1d_mfma_chunked_1x1(const ConvLaunch& a);
// Scratch floats a launch needs for split-K partial sums (0: no split).
size_t conv1d_mfma_split_floats(const ConvLaunch& a);
// Whether the launch, given post = POST_WN_GATE (post_H = C_out / 2), takes a
// path that applies the gate (split-K reduce or the small-conv kernel); the
// caller adds a separate gate launch otherwise.
bool conv1d_mfma_fuses_gate(const ConvLaunch& a);
// Whether the launch runs on the small-conv (whole-reduction) kernels, the
// only ones that take COMB_SUB.
bool conv1d_mfma_small_path(const ConvLaunch& a);
void launch_conv1d_mfma(const ConvLaunch& a, hipStream_t s);
// out = combine(act(sum of the split-K partials + bias ...)) for a launch
// with a.ksplit > 1 (shared by the fp32 and bf16 kernels)
void launch_splitk_reduce(const ConvLaunch& a, hipStream_t s);

// The bf16 variant (v_mfma_f32_32x32x16_bf16, fp32 accumulate, input stride 1):
// every group carries bf16 weights in g.w16 with row length a.w16_ld.
bool conv1d_bf16_supported(int K, int dil);
size_t conv1d_bf16_split_floats(const ConvLaunch& a);
void launch_conv1d_bf16(const ConvLaunch& a, hipStream_t s);
// bf16 weight row length for C_in input channels
inline int bf16_ld(int C_in) { return (C_in + 7) / 8 * 8; }
// device-side bf16 packers: [C_out][C_in][K] -> [K][C_out][bf16_ld(C_in)], and
// ConvTranspose phase r: [C_in][C_out][K] -> [J][C_out][bf16_ld(C_in)]
void launch_pack_conv_weight_bf16(const float* w, uint16_t* out, int C_out, int C_in, int K, hipStream_t s);
void launch_pack_convt_phase_bf16(const float* w, uint16_t* out, int C_in, int C_out, int K, int st, int r, int J,
                                  hipStream_t s);
// float -> bf16 bits, round to nearest even (the device staging uses the same rule)
inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// packed-weight leading dimension for C_out output channels
inline int packed_ld(int c_out) { return (c_out + 3) / 4 * 4; }

// Direct (vector ALU) conv1d for strided / tiny-channel shapes
// (noise convs, conv_post): out[b][co][i*out_step+out_off] from
// x[b][ci][i*stride + in_off + k*dil].
struct DirectConvArgs {
  const float* x; long long xb, xc;
  // x2, x3 (optional, same layout as x): the input is ((x + x2) + x3) / 3,
  // formed while staging (stride-1 launches with fewer than 8 outputs only)
  const float* x2; const float* x3;
  const float* w;  // PyTorch layout [C_out][C_in][K]
  const float* bias;
  float* out; long long ob, oc;
  int C_in, C_out, L_in, n_out, K, stride, dil, in_off;
  int in_act; float in_slope;
  int out_act; float out_slope;
  int combine; float div;
  int B;
};
void launch_conv1d_direct(const DirectConvArgs& a, hipStream_t s);

// ConvTranspose1d in gather form (any stride/padding/output_padding/dilation),
// weights in PyTorch layout [C_in][C_out][K]; bias added after the taps.
struct ConvTArgs {
  const float* x; long long xb, xc;
  const float* w;
  const float* bias;
  float* out; long long ob, oc;
  int C_in, C_out, L_in, n_out, K, stride, padding, dil;
  int in_act; float in_slope;
  int combine;
  int B;
  // Segment form: output index o is absolute column o + o_off of the full
  // transposed conv (written there, row stride oc), and only input columns
  // in [win_lo, win_lo + win_len) contribute (win_len == 0: the whole row).
  int o_off, win_lo, win_len;
};
void launch_conv_t1d_direct(const ConvTArgs& a, hipStream_t s);

// Polyphase ConvTranspose1d (dilation 1) on the MFMA kernel, all phases in
// one grouped launch; w_phases[r] holds the packed weights of phase r
// (launch_pack_convt_phase), ld packed_ld(C_out).  stride <= kMaxConvGroups.
void convt_polyphase(hipStream_t st, const float* x, long long xb, long long xc, const float* const* w_phases,
                     const float* bias, float* out, long long ob, long long oc, int B, int C_in, int C_out, int L,
                     int n_out, int K, int stride, int padding, int in_act, float in_slope, int combine,
                     int o_lo = 0, int x_shift = 0);
// The same with bf16 phase weights ([J_r][C_out][w16_ld] per phase) on the bf16 kernel.
void convt_polyphase_bf16(hipStream_t st, const float* x, long long xb, long long xc,
                          const uint16_t* const* w16_phases, int w16_ld, const float* bias, float* out, long long ob,
                          long long oc, int B, int C_in, int C_out, int L, int n_out, int K, int stride, int padding,
                          int in_act, float in_slope, int combine);
// (Segment form: only output columns [o_lo, n_out) are computed, and x's
// column 0 is input column x_shift of the full row, L its window length.)
// taps of phase r of a stride-st ConvTranspose with K taps
inline int convt_phase_taps(int K, int st, int r) { return r < K ? (K - r + st - 1) / st : 0; }

// Output-stationary polyphase ConvTranspose1d + bias + the NSF noise term
// (convt_os.hip):
//   out[b][co][o] = (sum_{ci,k} w[k][ci][co] lrelu(x[b][ci][m-j]) + bias[co]) + noise
//   with o + pad = m*S + r, k = r + j*S; noise = noise[b][co][o] when the
//   tensor is given, else (sum_{t<kn} nw[co][t] har[b][o*ns - np + t]) + nb[co].
constexpr int kNoiseTapsMax = 8;  // longest noise kernel computed in the epilogue
struct ConvTOsLaunch {
  const float* x; long long xb; int L_in;       // input [B][C_in][L_in]
  const float* w; int w_ld;                     // packed [K][C_in][w_ld], 16-byte rows
  const float* bias;                            // [C_out] or null
  float* out; long long ob, oc; int L_out;      // [B][C_out (stride oc)][L_out]
  int B, C_in, C_out, K, S, pad;
  int M;                                        // input positions covered: ceil((L_out + pad) / S)
  float in_slope;                               // leaky ReLU on the staged input
  const float* noise;                           // [B][C_out][L_out] (strides ob, oc) or null
  const float* har; long long harb; long long N;  // harmonic source [B][N]
  const float* nw; const float* nb; int kn, ns, np;  // noise conv [C_out][kn], [C_out]
  // bf16 operands (w16 set): weights [K][C_out][w16_ld] in bf16, the input
  // rounded to bf16 after the leaky ReLU, fp32 accumulate; w / w_ld unused
  const uint16_t* w16; int w16_ld;
};
// (K, S) shapes the kernel is instantiated for: (16, 10), (20, 10), (24, 12), (4, 2);
// the bf16 form needs C_in % 32 == 0 as well
bool convt_os_supported(int K, int S);
// false when no instantiation fits (C_out / C_in multiples)
bool launch_convt_os(const ConvTOsLaunch& a, hipStream_t s);

// Weight packing kernels (device side, used by the op-level ABI).
// [C_out][C_in][K] -> [K][C_in][packed_ld(C_out)] (pad columns zero)
void launch_pack_conv_weight(const float* w, float* out, int C_out, int C_in, int K, hipStream_t s);

// ---------------------------------------------------------------- fixed scratch (noalloc.hip)
// Per-GPU static device array behind the entry points that allocate nothing:
// 1 Mi floats (4 MiB).  noalloc_setup(device) looks up the array's address on
// `device` (which must be current) once; noalloc_scratch returns it.
constexpr size_t kNoAllocScratchFloats = (size_t)1 << 20;
void noalloc_setup(int device);
float* noalloc_scratch(int device);
// ConvTranspose [C_in][C_out][K], phase r of stride st with J taps:
// out[j'][ci][co] = w[ci][co][r + (J-1-j')*st], ld packed_ld(C_out)
void launch_pack_convt_phase(const float* w, float* out, int C_in, int C_out, int K, int st, int r,
                             int J, hipStream_t s);

// ---------------------------------------------------------------- elementwise
void launch_leaky(float* a, long long n, float slope, hipStream_t s);
void launch_relu(float* a, long long n, hipStream_t s);
void launch_copy(float* dst, const float* src, long long n, hipStream_t s);
void launch_add_inplace(float* a, const float* b, long long n, hipStream_t s);
void launch_mul_inplace(float* a, const float* b, long long n, hipStream_t s);
void launch_add(float* c, const float* a, const float* b, long long n, hipStream_t s);
void launch_mul(float* c, const float* a, const float* b, long long n, hipStream_t s);
void launch_fill(float* a, long long n, float v, hipStream_t s);
// out = a + gelu(p)
void launch_add_gelu(float* out, const float* a, const float* p, long long n, hipStream_t s);
// HuBERT's grouped long positional conv (posconv.hip): x, out [B][H][L],
// w [H / cpg][K][cpg (in)][cpg (out)], bias [H]; out[t] reads x[t + k - pad]
bool posconv_supported(int cpg, int K, int pad);
void launch_posconv(const float* x, const float* w, const float* bias, float* out, int B, int H, int L, int cpg,
                    int K, int pad, hipStream_t s);
// a = gelu(a) in place (erf form, gelu_as)
void launch_gelu(float* a, long long n, hipStream_t s);
// out[i] = a[i] + bias[i % cols]
void launch_bias_add(float* out, const float* a, const float* bias, long long n, long long cols, hipStream_t s);
// out = ((a + b) + c) / 3   (the ResBlock average, runtime/models/vits.py:2225-2227)
void launch_avg3(float* out, const float* a, const float* b, const float* c, long long n, hipStream_t s);
// out[i, :] = table[ids[i], :], ids int32 with negative wrap.
void launch_embed_i32(const int* ids, const float* table, float* out, long long n, int rows, int dim,
                      hipStream_t s);
// out[b][p][c] = src[b][c][p] * scale  (per batch, C x P -> P x C)
void launch_transpose(const float* src, float* out, int B, int C, int P, float scale, hipStream_t s);
// dst[b][c][t] = src[b][C-1-c][t]
void launch_flip_channels(const float* src, float* dst, int B, int C, int L, hipStream_t s);
// x[b][c][t] = lrelu((E[b][c][t] + table[pitch[b][t]][c]) * scale, slope); an id
// outside [-rows, rows) sets bit 0 of *err (nullable) and reads a clamped row
void launch_embed_combine(const float* E, const long long* pitch, const float* table, int rows, float* x,
                          int B, int C, int P, float scale, float slope, unsigned* err, hipStream_t s);
// acts[b][c][t] = tanh(a[c] + g[c]) * sigmoid(a[H+c] + g[H+c]), a = XI[b], g per batch [2H]
void launch_wn_gate(const float* XI, long long xib, const float* g, long long gb, float* acts, int B,
                    int H, int L, hipStream_t s);
// record/commit op 18: c[i] = tanh(a[i]+g1) * sigmoid(a[i+n]+g2)
void launch_gating(const float* a, const float* g, float* c, long long n, int lg, int h, long long off,
                   hipStream_t s);
// z[b][c][t] = m + exp(logs) * nz * k   with m = st[b][c], logs = st[b][H+c]
void launch_zp(const float* st, const float* nz, float* z, int B, int H, int L, float k, hipStream_t s);
// h[b][c][t] += rs[b][c][t] (c<H); skip[b][c][t] (=|+=) rs[b][H+c][t]
void launch_wn_update(float* h, float* skip, const float* rs, int B, int H, int L, int first,
                      int last, hipStream_t s);
// x1[b][c][t] = x1 - m   (x1 strided inside z)
void launch_sub_inplace_strided(float* x1, long long x1b, const float* m, long long mb, int B,
                                int C, int L, hipStream_t s);
// out[b][:] = table[clamp(ids[b])][:]  (int64 ids, negative wrap); an id outside
// [-rows, rows) sets bit 1 of *err (nullable)
void launch_gather_rows_i64(const long long* ids, const float* table, float* out, int B, int rows, int dim,
                            unsigned* err, hipStream_t s);
// out[b][co] = bias[co] + sum_ci W[co][ci] * g[b][ci]   (1x1 conv on a length-1 signal)
void launch_gemv(const float* W, const float* bias, const float* g, long long gb, float* out,
                 long long ob, int B, int C_out, int C_in, hipStream_t s);

// ---------------------------------------------------------------- NSF source
// Per-frame NSF phase of f0 [B][P]: out[b][p + shift] = rad_acc[b][p] (the
// reference's _phase_offsets for shift 0; for shift 1, out[b][0] = 0 and each
// frame gets the offset its phase adds).
void launch_sine_phase(const float* f0, float* out, int B, int P, int upp, float sr, int shift, hipStream_t s);
// har[b][p*upp+u] (see kernel docs).  seg_off [B][P] (nullable) holds every
// frame's whole phase offset (the reference's seg_offsets); without it the
// offsets come from f0's own cumulative phase, computed into off [B][P].
void launch_sine_source(const float* f0, const float* ns, float* har, float* off, const float* seg_off, int B,
                        int P, int upp, float sr, float w_lin, float b_lin, hipStream_t s);

// ---------------------------------------------------------------- norms
// Row-major LayerNorm over the last axis: x[rows][cols].
void launch_layernorm_rows(const float* x, const float* g, const float* b, float* out, long long rows,
                           int cols, float eps, hipStream_t s);
// Channel-major LayerNorm over C for each (b, t): x[b][C][L]
void launch_layernorm_cols(const float* x, const float* g, const float* b, float* out, int B, int C,
                           int L, float eps, hipStream_t s);
void launch_softmax_rows(const float* x, float* out, long long rows, int cols, hipStream_t s);
// One-channel-per-group GroupNorm over L of x[B][C][L], affine per channel, then act.
void launch_groupnorm_rows_act(const float* x, const float* g, const float* b, float* out, int B, int C, long long L,
                               float eps, int act, hipStream_t s);
// x [G][Cpg*S] standardised per row, affine of channel g*Cpg + i/S
void launch_groupnorm_groups(const float* x, const float* g, const float* b, float* out, long long G, int Cpg,
                             long long S, float eps, hipStream_t s);
// out = x / sqrt(mean(x^2) + eps) * gamma, per row of [rows][cols]
void launch_rmsnorm_rows(const float* x, const float* g, float* out, long long rows, int cols, float eps,
                         hipStream_t s);

// ---------------------------------------------------------------- attention
// Windowed relative-position attention, all heads (emb_k = emb_v = null:
// plain attention).
// qkv[b][3*H*D][P] (q, k, v stacked), emb_k/emb_v [2w+1][D], out[b][H*D][P];
// scratch (scratch_floats floats) must hold
// relpos_attention_scratch_floats(B,H,D,P,window,band) floats (band: emb_k
// given; may be null when that is 0); a smaller buffer is an error.
void launch_relpos_attention(const float* qkv, const float* emb_k, const float* emb_v, float* out,
                             float* scratch, size_t scratch_floats, int B, int H, int D, int P, int window,
                             hipStream_t s);
size_t relpos_attention_scratch_floats(int B, int H, int D, int P, int window, bool band);
size_t relpos_attention_max_frames();
// The key split the attention kernel uses for (H, D, P, window); a function
// of the shape only, never of B.
int relpos_attention_splits(int H, int D, int P, int window, bool band);
// The attention kernel alone, without the merge launch: returns the key
// split KS.  KS == 1: out holds the attention output; KS > 1: scratch holds
// the partials part[b][h][ks] = (m[P], l[P], O[D][P]) for a consumer that
// merges them (launch_attn_out_ln).
int launch_relpos_attention_partials(const float* qkv, const float* emb_k, const float* emb_v, float* out,
                                     float* scratch, size_t scratch_floats, int B, int H, int D, int P, int window,
                                     hipStream_t s);

// enc_p's attention output block in one launch (attn_out.hip): merge of the
// attention partials (KS > 1) or the merged output (KS == 1), conv_o + bias,
// + the residual, LayerNorm over the C = H * D channels.  Tensors [B][C][P]
// contiguous; w in SessionBase::pack_mfma_lanes order.
struct AttnOutArgs {
  const float* part;  // KS > 1
  const float* att;   // KS == 1
  const float* w;
  const float* bias;
  const float* res;
  const float* g;
  const float* beta;
  float* out;
  int H, D, P, KS;
  float eps;
};
bool attn_out_ln_supported(int H, int D, int KS);
void launch_attn_out_ln(const AttnOutArgs& a, int B, hipStream_t s);

// The end of a reverse flow and the next flow's pre conv in one launch
// (flow_tail.hip): skip' = skip + (W_rs acts + b_rs); x1 -= W_post skip' +
// b_post; h = W_pre x1 + b_pre (skipped when w_pre is null).  acts, skip, h
// [B][C][P] contiguous; x1 [HALF = C / 2][P] at batch stride xb; weights in
// SessionBase::pack_mfma_lanes order.
struct FlowTailArgs {
  const float* acts;
  const float* skip;
  const float* w_rs;
  const float* b_rs;
  const float* w_post;
  const float* b_post;
  float* x1;
  long long xb;
  const float* w_pre;
  const float* b_pre;
  float* h;
  int P;
};
bool flow_tail_supported(int C, int half);
void launch_flow_tail(const FlowTailArgs& a, int C, int B, hipStream_t s);

// Op-level attention on head-interleaved [T][C] q/k/v (head h in columns
// [h*D, (h+1)*D)); used [2T-1][D] (relative table, m = s - t + T - 1) or null.
//   scores [H][T][T] = q_h . (k_h + used[m])
//   ctx [T][C]       = sum_s W[h][t][s] (v_h[s] + used[m])
void launch_attn_scores(const float* q, const float* k, const float* used, float* out, int H, int T, int D, int C,
                        hipStream_t s);
void launch_attn_context(const float* w, const float* v, const float* used, float* out, int H, int T, int D, int C,
                         hipStream_t s);

// ---------------------------------------------------------------- matmul
// c[M][N] = a[M][K] @ b[K][N], row-major (op-level rvc_matmul)
void launch_matmul(const float* a, const float* b, float* c, int M, int K, int N, hipStream_t s);

// ------------------------------------------------------------------ conv2d
// Implicit-GEMM 2-D convolution on fp32 MFMA (csrc/rmvpe.hip).  Computed
// point (a, b) of group g (a < oh_n <= OH, b < ow_n <= OW) sums, over taps t and input
// channels ci, w_t[ci][co] * x[ci][a*stride + dh_t][b*stride + dw_t] (zero
// outside [0, H) x [0, W)); points with a >= a_lim or b >= b_lim take no taps.
// v = acc + bias; relu; + res; stored at
//   out[b*ob + co*oc + (a*osh + oh0)*ors + (b*osw + ow0)*ocs]  (res alike).
constexpr int kConv2dTapsMax = 9;
constexpr int kConv2dGroupsMax = 4;
struct Conv2dGroup {
  const float* w;  // packed [ntaps][C_in][w_ld], 16-byte aligned
  int ntaps;
  int dh[kConv2dTapsMax], dw[kConv2dTapsMax];
  int oh0, ow0;
  int a_lim, b_lim;
  int oh_n, ow_n;  // this group's computed extent (<= OH, OW); points beyond it are not stored
  int dh_lo, dw_lo, dh_span, dw_span;  // set by the launcher
};
struct Conv2dLaunch {
  Conv2dGroup g[kConv2dGroupsMax];
  int n_groups;
  const float* x; long long xb, xc; int H, W;   // input [B][C_in (stride xc)][H][W]
  float* out; long long ob, oc, ors, ocs;
  const float* res;
  const float* bias;
  int relu;
  int C_in, C_out, w_ld, B;
  int OH, OW, osh, osw;
  int stride;                                   // 1 or 2 on both axes
  float* part; size_t part_floats;              // split-K scratch (optional)
  int ksplit, csplit, tile_c;                   // set by the launcher
};
size_t conv2d_split_floats(const Conv2dLaunch& a);
void launch_conv2d(const Conv2dLaunch& a, hipStream_t s);
// host-side packing: [C_out][C_in][KH][KW] (times scale[co] when given) ->
// [KH*KW][C_in][packed_ld(C_out)], tap t = kh*KW + kw
std::vector<float> pack_conv2d_host(const float* w, const float* scale, int C_out, int C_in, int KH, int KW);
void launch_pack_conv2d_weight(const float* w, float* out, int C_out, int C_in, int KH, int KW, hipStream_t s);
// ConvTranspose2d weights w [C_in][C_out][KH][KW] -> [ntaps][C_in][packed_ld(C_out)] for the taps (kh[t], kw[t])
// of one stride phase (kh[t] < 0: an all-zero tap)
struct ConvT2dTaps {
  int n;
  int kh[kConv2dTapsMax], kw[kConv2dTapsMax];
};
void launch_pack_convt2d_phase(const float* w, float* out, int C_in, int C_out, int KH, int KW, const ConvT2dTaps& t,
                               hipStream_t s);
void launch_insert_zeros_2x(const float* x, float* out, long long C, int H, int W, hipStream_t s);
void launch_avg_pool2(const float* x, float* out, int BC, int H, int W, hipStream_t s);

// ------------------------------------------------------------------ RMVPE
void launch_rmvpe_blocks(const float* x, int T, float* xb, int NB, hipStream_t s);
void launch_mel_mag(const float* S, float* mag, int nbin, int F, hipStream_t s);
void launch_logmel_image(const float* M, int F, int Fp, int n_mels, float bn_s, float bn_t, float* img,
                         float* logmel, hipStream_t s);
struct GruArgs {
  const float* gx;  long long g_d, g_t, g_r;   // gate input of (direction, step, gate row)
  const float* whh; const float* bhh;          // [2][3H][H], [2][3H]
  float* out;       long long o_d, o_t, o_j;   // h of (direction, step, unit)
  unsigned long long* state;                    // [2][2][256] tagged hidden-state double buffer
  unsigned* sync;                               // [4]: arrivals per direction, error flag
  int T, H;
  long long spin_limit;
  int keep_err;  // 1: leave the error flag as an earlier, unchecked GRU left it
};
void launch_bigru(const GruArgs& g, hipStream_t s);
void launch_rmvpe_decode(const float* sal, long long s_f, long long s_k, int F, int nb, const float* cents,
                         float thred, float* f0, hipStream_t s);

}  // namespace rvc
