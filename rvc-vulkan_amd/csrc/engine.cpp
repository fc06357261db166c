// The C ABI of the HIP backend: engine / memory / single-op / record-commit
// exports with the reference's names, argument meaning and error convention
// (engine/src/ffi.zig:1-1119): every export returns int32 0 on success and
// -1 on failure with the message in a process-global, mutex-protected
// buffer read by rvc_last_error; rvc_engine_create returns an int64 handle
// or -1; buffer ids are opaque int64 keys, 0 meaning "no bias"; sizes are
// float counts except rvc_mem_alloc / rvc_mem_fill_zero (bytes); f32
// scalars travel as IEEE bit patterns in int64 (slope, batch eps, scale).
// Every call on an engine is serialised by its mutex.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>

#include "../../include/rvc_hip.h"
#include "engine.h"

namespace rvc {

// ---------------------------------------------------------------- errors
namespace {
std::mutex g_err_mu;
std::string g_err;
std::mutex g_tab_mu;
std::unordered_map<long long, Engine*> g_engines;
long long g_next_handle = 1;
long long g_last_engine = 0;
}  // namespace

void set_last_error(const std::string& msg) {
  std::lock_guard<std::mutex> lk(g_err_mu);
  g_err = msg.substr(0, 4095);
}

void check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) throw Error(std::string(what) + " launch failed: " + hipGetErrorString(e));
}

StopHook& stop_hook() {
  static thread_local StopHook h;
  return h;
}

Engine* engine_from_handle(long long h) {
  std::lock_guard<std::mutex> lk(g_tab_mu);
  auto it = g_engines.find(h);
  return it == g_engines.end() ? nullptr : it->second;
}

Engine::Engine() {
  int n = 0;
  RVC_HIP(hipGetDeviceCount(&n));
  RVC_CHECK(n > 0, "no HIP device");
  RVC_HIP(hipGetDevice(&device));
  hipDeviceProp_t prop;
  RVC_HIP(hipGetDeviceProperties(&prop, device));
  // some drivers leave the marketing name empty; the ISA name is always set
  const std::string nm = prop.name[0] ? std::string(prop.name) : std::string("AMD GPU");
  device_name = nm + " (" + prop.gcnArchName + ", " + std::to_string(prop.multiProcessorCount) + " CUs)";
  RVC_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
  noalloc_setup(device);
  const char* ts = std::getenv("RVC_TS");
  ts_on = ts && std::strcmp(ts, "1") == 0;
}

Engine::~Engine() {
  if (stream) (void)hipStreamSynchronize(stream);
  for (auto& ev : ts_pending) (void)hipEventDestroy(ev.first), (void)hipEventDestroy(ev.second);
  for (auto& kv : bufs) (void)hipFree(kv.second.ptr);
  if (scratch) (void)hipFree(scratch);
  if (stream) (void)hipStreamDestroy(stream);
}

long long Engine::add_buffer(void* p, size_t bytes) {
  const long long id = next_id++;
  bufs[id] = DevBuf{p, bytes};
  return id;
}

DevBuf& Engine::get(long long id) {
  auto it = bufs.find(id);
  if (it == bufs.end()) throw Error("invalid buffer id " + std::to_string(id));
  return it->second;
}

float* Engine::fptr(long long id, long long n_floats, const char* what) {
  DevBuf& b = get(id);
  if (n_floats < 0 || (size_t)n_floats * sizeof(float) > b.bytes)
    throw Error(std::string(what) + ": buffer " + std::to_string(id) + " holds " +
                std::to_string(b.bytes / sizeof(float)) + " floats, needs " + std::to_string(n_floats));
  return static_cast<float*>(b.ptr);
}

void* Engine::scratch_for(size_t bytes) {
  if (bytes > scratch_bytes) {
    RVC_HIP(hipStreamSynchronize(stream));
    if (scratch) RVC_HIP(hipFree(scratch));
    scratch = nullptr;
    scratch_bytes = 0;
    RVC_HIP(hipMalloc(&scratch, bytes));
    scratch_bytes = bytes;
  }
  return scratch;
}

void Engine::sync() { RVC_HIP(hipStreamSynchronize(stream)); }

void Engine::ts_collect() {
  sync();
  for (auto& ev : ts_pending) {
    float ms = 0.f;
    const hipError_t er = hipEventElapsedTime(&ms, ev.first, ev.second);
    (void)hipEventDestroy(ev.first);
    (void)hipEventDestroy(ev.second);
    if (er == hipSuccess) ts_busy_ns += (long long)((double)ms * 1e6);
  }
  ts_pending.clear();
}

// Run one submission; with RVC_TS=1 it is bracketed by events on the stream.
template <class F>
static void submit(Engine& e, F&& f) {
  if (!e.ts_on) {
    f();
    return;
  }
  hipEvent_t a, b;
  RVC_HIP(hipEventCreate(&a));
  if (hipEventCreate(&b) != hipSuccess) {
    (void)hipEventDestroy(a);
    throw Error("hipEventCreate failed");
  }
  e.ts_pending.push_back({a, b});
  RVC_HIP(hipEventRecord(a, e.stream));
  f();
  RVC_HIP(hipEventRecord(b, e.stream));
  ++e.ts_submits;
}

// ---------------------------------------------------------------- ops
// Every op checks its parameters and buffers first and launches only when
// `dry` is false.  The record calls of the batch API run the op with
// dry = true, so a bad record fails at rvc_batch_add* (the reference checks
// at record time too, engine/src/engine.zig:2078-2094), and the commit
// launches.
namespace {

float bits_to_f32(long long v) {
  const uint32_t u = (uint32_t)((unsigned long long)v & 0xffffffffULL);
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// Floats [off, off + n) of buffer `id`, checked against its size.
float* fview(Engine& e, long long id, long long off, long long n, const char* what) {
  RVC_CHECK(off >= 0 && n >= 0, std::string(what) + ": negative offset or size");
  return e.fptr(id, off + n, what) + off;
}

// A byte offset of a sub-view (-1: none) as a float offset.
long long view_floats(long long bytes, const char* what) {
  if (bytes < 0) return 0;
  RVC_CHECK(bytes % 4 == 0, std::string(what) + ": view offset must be a multiple of 4 bytes");
  return bytes / 4;
}

void check_i32(long long v, const char* what) {
  RVC_CHECK(v >= 0 && v <= 0x7fffffffLL, std::string(what) + ": dimension exceeds 32-bit indexing");
}

// A one-group MFMA launch over x [B][C_in][L] -> out [B][C_out][n_out].
ConvLaunch one_conv(const float* x, long long C_in, long long L, const float* packed, const float* bias, float* out,
                    long long C_out, long long n_out, long long B, long long K, long long dil, long long pad_l,
                    long long stride = 1) {
  ConvLaunch a{};
  a.n_groups = 1;
  ConvGroup& g = a.g[0];
  g.x = x; g.w = packed; g.bias = bias; g.res = nullptr; g.out = out;
  g.K = (int)K; g.dil = (int)dil; g.in_off = (int)-pad_l; g.in_step = (int)stride; g.out_step = 1; g.out_off = 0;
  g.n_out = (int)n_out; g.combine = COMB_STORE;
  a.xb = C_in * L; a.xc = L; a.ob = C_out * n_out; a.oc = n_out;
  a.C_in = (int)C_in; a.C_out = (int)C_out; a.w_ld = packed_ld((int)C_out); a.L_in = (int)L; a.B = (int)B;
  a.div = 1.f;
  return a;
}

// Output columns [lo_off, lo_off + n_seg) of the conv1d
//   out[b][co][o] = bias[co] + sum_{ci,k} w[co][ci][k] x[b][ci][o*stride - pad_l + k*dil]
// (zero outside [0, L)), written into rows of length row_len.
// fixed_packed (nullable): where the fp32 MFMA path packs the weights,
// holding fixed_floats floats, instead of the engine's growable scratch.
void conv1d_core(Engine& e, bool dry, long long x, long long w, long long b, long long out, long long B,
                 long long C_in, long long L, long long C_out, long long K, long long stride, long long pad_l,
                 long long dil, long long n_seg, long long lo_off, long long row_len, bool bf16 = false,
                 float* fixed_packed = nullptr, size_t fixed_floats = 0) {
  RVC_CHECK(n_seg >= 1 && lo_off >= 0 && lo_off + n_seg <= row_len, "conv1d: output segment outside the output row");
  check_i32(L, "conv1d"); check_i32(row_len, "conv1d"); check_i32(lo_off * stride + pad_l, "conv1d");
  check_i32(C_in * K, "conv1d"); check_i32(C_out, "conv1d");
  const float* xp = e.fptr(x, B * C_in * L, "conv1d x");
  const float* wp = e.fptr(w, C_out * C_in * K, "conv1d w");
  const float* bp = b ? e.fptr(b, C_out, "conv1d bias") : nullptr;
  float* op = e.fptr(out, (B * C_out - 1) * row_len + lo_off + n_seg, "conv1d out");
  if (bf16)
    RVC_CHECK(stride == 1 && conv1d_bf16_supported((int)K, (int)dil),
              "conv1d_bf16: stride 1, K <= " + std::to_string(kConvTapsMax) + " and (K-1)*dil <= " +
                  std::to_string(kConvHaloMax) + " only");
  const bool mfma = !bf16 && (stride == 1 || stride == 2) && conv1d_mfma_supported((int)K, (int)dil);
  const size_t packed_floats = (size_t)packed_ld((int)C_out) * C_in * K;
  if (fixed_packed && mfma)
    RVC_CHECK(packed_floats <= fixed_floats,
              "conv1d_noalloc: the packed weights need " + std::to_string(packed_floats) +
                  " floats (packed_ld(C_out) * C_in * K); the fixed scratch holds " + std::to_string(fixed_floats));
  if (dry) return;
  const long long in_off = lo_off * stride - pad_l;
  if (bf16) {
    uint16_t* packed = static_cast<uint16_t*>(e.scratch_for(sizeof(uint16_t) * K * C_out * bf16_ld((int)C_in)));
    launch_pack_conv_weight_bf16(wp, packed, (int)C_out, (int)C_in, (int)K, e.stream);
    ConvLaunch a = one_conv(xp, C_in, L, nullptr, bp, op, C_out, n_seg, B, K, dil, pad_l, 1);
    a.g[0].w16 = packed;
    a.w16_ld = bf16_ld((int)C_in);
    a.g[0].in_off = (int)in_off;
    a.g[0].out_off = (int)lo_off;
    a.ob = C_out * row_len;
    a.oc = row_len;
    launch_conv1d_bf16(a, e.stream);
  } else if (mfma) {
    float* packed = fixed_packed ? fixed_packed : static_cast<float*>(e.scratch_for(sizeof(float) * packed_floats));
    launch_pack_conv_weight(wp, packed, (int)C_out, (int)C_in, (int)K, e.stream);
    ConvLaunch a = one_conv(xp, C_in, L, packed, bp, op, C_out, n_seg, B, K, dil, pad_l, stride);
    a.g[0].in_off = (int)in_off;
    a.g[0].out_off = (int)lo_off;
    a.ob = C_out * row_len;
    a.oc = row_len;
    launch_conv1d_mfma(a, e.stream);
  } else {
    DirectConvArgs a{};
    a.x = xp; a.xb = C_in * L; a.xc = L;
    a.w = wp; a.bias = bp;
    a.out = op + lo_off; a.ob = C_out * row_len; a.oc = row_len;
    a.C_in = (int)C_in; a.C_out = (int)C_out; a.L_in = (int)L; a.n_out = (int)n_seg;
    a.K = (int)K; a.stride = (int)stride; a.dil = (int)dil; a.in_off = (int)in_off;
    a.combine = COMB_STORE; a.div = 1.f; a.B = (int)B;
    launch_conv1d_direct(a, e.stream);
  }
}

void op_conv1d(Engine& e, bool dry, long long x, long long w, long long b, long long out, long long B,
               long long C_in, long long L, long long C_out, long long K, long long stride, long long pad_l,
               long long pad_r, long long dil, bool bf16 = false, float* fixed_packed = nullptr,
               size_t fixed_floats = 0) {
  RVC_CHECK(B >= 1 && C_in >= 1 && C_out >= 1 && K >= 1 && stride >= 1 && dil >= 1 && pad_l >= 0 &&
                pad_r >= 0 && L >= 0,
            "conv1d: invalid parameters (stride/dilation>=1, padding>=0, K>=1)");
  const long long n_out = (L + pad_l + pad_r - dil * (K - 1) - 1) / stride + 1;
  RVC_CHECK(L + pad_l + pad_r - dil * (K - 1) - 1 >= 0 && n_out >= 1, "conv1d: empty output");
  conv1d_core(e, dry, x, w, b, out, B, C_in, L, C_out, K, stride, pad_l, dil, n_out, 0, n_out, bf16, fixed_packed,
              fixed_floats);
}

// engine/src/ffi.zig:703-751: the output segment [lo_off, lo_off + seg_len)
// of a conv1d with symmetric padding, rows of length l_out_full.
void op_conv1d_seg(Engine& e, bool dry, long long x, long long w, long long b, long long out, long long B,
                   long long C_in, long long L, long long C_out, long long K, long long stride, long long pad_l,
                   long long pad_r, long long dil, long long seg_len, long long lo_off, long long l_out_full) {
  RVC_CHECK(B >= 1 && C_in >= 1 && L >= 1 && C_out >= 1 && K >= 1 && stride >= 1 && dil >= 1 && pad_l >= 0,
            "conv1d_seg: invalid parameters");
  RVC_CHECK(pad_r == pad_l, "conv1d_seg: the segmented conv1d needs symmetric padding (pad_r == pad_l)");
  conv1d_core(e, dry, x, w, b, out, B, C_in, L, C_out, K, stride, pad_l, dil, seg_len, lo_off, l_out_full);
}

// The grouped launch of a polyphase ConvTranspose1d (fp32 or bf16 phase weights).
ConvLaunch convt_polyphase_launch(const float* x, long long xb, long long xc, const float* const* w_phases,
                                  const uint16_t* const* w16_phases, const float* bias, float* out, long long ob,
                                  long long oc, int B, int C_in, int C_out, int L, int n_out, int K, int stride,
                                  int padding, int in_act, float in_slope, int combine, int o_lo, int x_shift) {
  RVC_CHECK(stride >= 1 && stride <= kMaxConvGroups, "conv_transpose1d: stride exceeds the grouped launch");
  ConvLaunch a{};
  a.xb = xb; a.xc = xc; a.ob = ob; a.oc = oc;
  a.C_in = C_in; a.C_out = C_out; a.w_ld = packed_ld(C_out); a.L_in = L; a.B = B;
  a.in_act = in_act; a.in_slope = in_slope; a.div = 1.f;
  for (int r = 0; r < stride; ++r) {
    const int J = convt_phase_taps(K, stride, r);
    // m range with o_lo <= m*stride + r - padding < n_out
    const int lo = o_lo + padding - r;
    const int m0 = lo <= 0 ? 0 : (lo + stride - 1) / stride;
    const int hi = n_out - 1 - r + padding;
    if (hi < 0) continue;
    const int m1 = hi / stride;
    if (m1 < m0) continue;
    ConvGroup& g = a.g[a.n_groups++];
    g.x = x; g.bias = bias; g.res = nullptr; g.out = out;
    g.w = w_phases ? w_phases[r] : nullptr;
    g.w16 = w16_phases ? w16_phases[r] : nullptr;
    g.K = J; g.dil = 1; g.in_off = m0 - (J > 0 ? J - 1 : 0) - x_shift;
    g.out_step = stride; g.out_off = m0 * stride + r - padding;
    g.n_out = m1 - m0 + 1; g.combine = combine;
  }
  return a;
}

}  // namespace

// Polyphase ConvTranspose1d on the MFMA kernel (dilation 1): output o with
// (o + padding) = m*stride + r only sees taps k = r + j*stride of input
// m - j, so phase r is a stride-1 conv over m with J_r taps whose outputs land
// at o = m*stride + r - padding.  All phases go into one grouped launch.
// Shared by the op-level exports and the synthesis session.
void convt_polyphase(hipStream_t st, const float* x, long long xb, long long xc, const float* const* w_phases,
                     const float* bias, float* out, long long ob, long long oc, int B, int C_in, int C_out, int L,
                     int n_out, int K, int stride, int padding, int in_act, float in_slope, int combine, int o_lo,
                     int x_shift) {
  const ConvLaunch a = convt_polyphase_launch(x, xb, xc, w_phases, nullptr, bias, out, ob, oc, B, C_in, C_out, L,
                                              n_out, K, stride, padding, in_act, in_slope, combine, o_lo, x_shift);
  if (a.n_groups > 0) launch_conv1d_mfma(a, st);
}

void convt_polyphase_bf16(hipStream_t st, const float* x, long long xb, long long xc,
                          const uint16_t* const* w16_phases, int w16_ld, const float* bias, float* out, long long ob,
                          long long oc, int B, int C_in, int C_out, int L, int n_out, int K, int stride, int padding,
                          int in_act, float in_slope, int combine) {
  ConvLaunch a = convt_polyphase_launch(x, xb, xc, nullptr, w16_phases, bias, out, ob, oc, B, C_in, C_out, L, n_out,
                                        K, stride, padding, in_act, in_slope, combine, 0, 0);
  a.w16_ld = w16_ld;
  if (a.n_groups > 0) launch_conv1d_bf16(a, st);
}

namespace {

// Output columns [lo_off, lo_off + n_seg) of the ConvTranspose1d
//   out[b][co][o] = bias[co] + sum_{k, i: i*stride - padding + k*dil = o} sum_ci x[b][ci][i] w[ci][co][k]
// where only input columns i in [win_lo, win_lo + win_len) contribute;
// rows of x have length L, rows of out length row_len; vx..vo are float
// offsets of sub-views into the four buffers.
void conv_t1d_core(Engine& e, bool dry, long long x, long long w, long long b, long long out, long long vx,
                   long long vw, long long vb, long long vo, long long B, long long C_in, long long L, long long C_out,
                   long long K, long long stride, long long padding, long long dil, long long n_seg, long long lo_off,
                   long long row_len, long long win_lo, long long win_len, bool bf16 = false) {
  RVC_CHECK(n_seg >= 1 && lo_off >= 0 && lo_off + n_seg <= row_len,
            "conv_transpose1d: output segment outside the output row");
  RVC_CHECK(win_lo >= 0 && win_len >= 1 && win_lo + win_len <= L,
            "conv_transpose1d: input window outside the input row");
  check_i32(L, "conv_transpose1d"); check_i32(row_len + padding + dil * K, "conv_transpose1d");
  check_i32(C_in, "conv_transpose1d"); check_i32(C_out, "conv_transpose1d");
  const float* xp = fview(e, x, vx, (B * C_in - 1) * L + win_lo + win_len, "conv_t1d x");
  const float* wp = fview(e, w, vw, C_in * C_out * K, "conv_t1d w");
  const float* bp = b ? fview(e, b, vb, C_out, "conv_t1d bias") : nullptr;
  float* op = fview(e, out, vo, (B * C_out - 1) * row_len + lo_off + n_seg, "conv_t1d out");
  const bool poly = dil == 1 && stride <= kMaxConvGroups && (K + stride - 1) / stride <= kConvTapsMax;
  if (bf16)
    RVC_CHECK(poly && lo_off == 0 && n_seg == row_len && win_lo == 0 && win_len == L,
              "conv_t1d_bf16: dilation 1, stride <= " + std::to_string(kMaxConvGroups) + " and ceil(K/stride) <= " +
                  std::to_string(kConvTapsMax) + " only");
  if (dry) return;
  const int ld = packed_ld((int)C_out);
  if (bf16) {
    const int ldi = bf16_ld((int)C_in);
    uint16_t* packed = static_cast<uint16_t*>(e.scratch_for(sizeof(uint16_t) * C_out * ldi * (K + stride)));
    std::vector<const uint16_t*> phases(stride);
    long long off = 0;
    for (int r = 0; r < stride; ++r) {
      const int J = convt_phase_taps((int)K, (int)stride, r);
      launch_pack_convt_phase_bf16(wp, packed + off, (int)C_in, (int)C_out, (int)K, (int)stride, r, J, e.stream);
      phases[r] = packed + off;
      off += (long long)J * C_out * ldi;
    }
    convt_polyphase_bf16(e.stream, xp, C_in * L, L, phases.data(), ldi, bp, op, C_out * row_len, row_len, (int)B,
                         (int)C_in, (int)C_out, (int)L, (int)n_seg, (int)K, (int)stride, (int)padding, ACT_NONE, 0.f,
                         COMB_STORE);
  } else if (poly) {
    // packed phases back to back in the scratch (16-byte aligned: ld % 4 == 0)
    float* packed = static_cast<float*>(e.scratch_for(sizeof(float) * C_in * ld * (K + stride)));
    std::vector<const float*> phases(stride);
    long long off = 0;
    for (int r = 0; r < stride; ++r) {
      const int J = convt_phase_taps((int)K, (int)stride, r);
      launch_pack_convt_phase(wp, packed + off, (int)C_in, (int)C_out, (int)K, (int)stride, r, J, e.stream);
      phases[r] = packed + off;
      off += (long long)J * C_in * ld;
    }
    convt_polyphase(e.stream, xp + win_lo, C_in * L, L, phases.data(), bp, op, C_out * row_len, row_len, (int)B,
                    (int)C_in, (int)C_out, (int)win_len, (int)(lo_off + n_seg), (int)K, (int)stride, (int)padding,
                    ACT_NONE, 0.f, COMB_STORE, (int)lo_off, (int)win_lo);
  } else {
    ConvTArgs a{};
    a.x = xp; a.xb = C_in * L; a.xc = L;
    a.w = wp; a.bias = bp;
    a.out = op; a.ob = C_out * row_len; a.oc = row_len;
    a.C_in = (int)C_in; a.C_out = (int)C_out; a.L_in = (int)L; a.n_out = (int)n_seg;
    a.K = (int)K; a.stride = (int)stride; a.padding = (int)padding; a.dil = (int)dil;
    a.combine = COMB_STORE; a.B = (int)B;
    a.o_off = (int)lo_off; a.win_lo = (int)win_lo; a.win_len = (int)win_len;
    launch_conv_t1d_direct(a, e.stream);
  }
}

void op_conv_t1d(Engine& e, bool dry, long long x, long long w, long long b, long long out, long long B,
                 long long C_in, long long L, long long C_out, long long K, long long stride, long long padding,
                 long long opad, long long dil, bool bf16 = false) {
  RVC_CHECK(B >= 1 && C_in >= 1 && C_out >= 1 && K >= 1 && stride >= 1 && dil >= 1 && padding >= 0 &&
                opad >= 0 && L >= 1,
            "conv_transpose1d: invalid parameters (stride/dilation>=1, padding/output_padding>=0)");
  const long long n_out = (L - 1) * stride - 2 * padding + dil * (K - 1) + opad + 1;
  RVC_CHECK(n_out >= 1, "conv_transpose1d: empty output");
  conv_t1d_core(e, dry, x, w, b, out, 0, 0, 0, 0, B, C_in, L, C_out, K, stride, padding, dil, n_out, 0, n_out, 0, L,
                bf16);
}

// engine/src/ffi.zig:636-701 (engine/src/engine.zig:2430-2468): output
// columns [lo_off, lo_off + l_out) of the transposed conv, input window
// [in_off, in_off + l_in_seg), byte-offset sub-views (-1: none).
void op_conv_t1d_seg(Engine& e, bool dry, const long long* p) {
  // p: a b c | B C_in L C_out K stride padding opad dil out | l_out l_in_seg in_off lo_off l_out_full | vx vw vb vo
  const long long x = p[0], w = p[1], b = p[2];
  const long long B = p[3], C_in = p[4], L = p[5], C_out = p[6], K = p[7], stride = p[8], padding = p[9],
                  dil = p[11], out = p[12];
  const long long l_out = p[13], l_in_seg = p[14], in_off = p[15], lo_off = p[16], l_out_full = p[17];
  RVC_CHECK(B >= 1 && C_in >= 1 && L >= 1 && C_out >= 1 && K >= 1 && stride >= 1 && dil >= 1 && padding >= 0 &&
                p[10] >= 0,
            "conv_t1d_seg: invalid parameters");
  conv_t1d_core(e, dry, x, w, b, out, view_floats(p[18], "conv_t1d_seg x"), view_floats(p[19], "conv_t1d_seg w"),
                view_floats(p[20], "conv_t1d_seg bias"), view_floats(p[21], "conv_t1d_seg out"), B, C_in, L, C_out, K,
                stride, padding, dil, l_out, lo_off, l_out_full, in_off, l_in_seg);
}

void op_matmul(Engine& e, bool dry, long long a, long long b, long long c, long long M, long long K, long long N) {
  RVC_CHECK(M >= 1 && K >= 1 && N >= 1, "matmul: invalid shape");
  check_i32(M, "matmul"); check_i32(K, "matmul"); check_i32(N, "matmul");
  const float* ap = e.fptr(a, M * K, "matmul a");
  const float* bp = e.fptr(b, K * N, "matmul b");
  float* cp = e.fptr(c, M * N, "matmul c");
  if (dry) return;
  // c[M][N] = a[M][K] b[K][N] as a 1x1 conv: channels = K, time = N; the
  // packed weights are a^T (a seen as a [M][K][1] conv weight).
  float* at = static_cast<float*>(e.scratch_for(sizeof(float) * packed_ld((int)M) * K));
  launch_pack_conv_weight(ap, at, (int)M, (int)K, 1, e.stream);
  launch_conv1d_mfma(one_conv(bp, K, N, at, nullptr, cp, M, N, 1, 1, 1, 0), e.stream);
}

void op_layernorm(Engine& e, bool dry, long long x, long long g, long long b, long long out, long long rows,
                  long long cols, float eps) {
  RVC_CHECK(rows >= 0 && cols >= 1, "layer_norm: invalid shape");
  check_i32(cols, "layer_norm");
  const float* xp = e.fptr(x, rows * cols, "layer_norm x");
  const float* gp = e.fptr(g, cols, "layer_norm gamma");
  const float* bp = e.fptr(b, cols, "layer_norm beta");
  float* op = e.fptr(out, rows * cols, "layer_norm out");
  if (!dry) launch_layernorm_rows(xp, gp, bp, op, rows, (int)cols, eps, e.stream);
}

void op_rmsnorm(Engine& e, bool dry, long long x, long long g, long long out, long long rows, long long cols,
                float eps) {
  RVC_CHECK(rows >= 0 && cols >= 1, "rmsnorm: invalid shape");
  check_i32(cols, "rmsnorm");
  const float* xp = e.fptr(x, rows * cols, "rmsnorm x");
  const float* gp = e.fptr(g, cols, "rmsnorm gamma");
  float* op = e.fptr(out, rows * cols, "rmsnorm out");
  if (!dry) launch_rmsnorm_rows(xp, gp, op, rows, (int)cols, eps, e.stream);
}

void op_softmax(Engine& e, bool dry, long long x, long long out, long long rows, long long cols) {
  RVC_CHECK(rows >= 0 && cols >= 1, "softmax: invalid shape");
  check_i32(cols, "softmax");
  const float* xp = e.fptr(x, rows * cols, "softmax x");
  float* op = e.fptr(out, rows * cols, "softmax out");
  if (!dry) launch_softmax_rows(xp, op, rows, (int)cols, e.stream);
}

void op_gating(Engine& e, bool dry, long long a, long long b, long long c, long long n, long long lg, long long h,
               long long off) {
  RVC_CHECK(n >= 1 && h >= 1 && n % h == 0 && (lg == 1 || lg == n / h) && off >= 0, "gating: invalid parameters");
  const float* ap = e.fptr(a, 2 * n, "gating a");
  const float* gp = e.fptr(b, off + 2 * h * lg, "gating g");
  float* cp = e.fptr(c, n, "gating out");
  if (!dry) launch_gating(ap, gp, cp, n, (int)lg, (int)h, off, e.stream);
}

void op_transpose(Engine& e, bool dry, long long a, long long c, long long C, long long P, float scale) {
  RVC_CHECK(C >= 1 && P >= 1, "transpose: invalid shape");
  check_i32(C, "transpose"); check_i32(P, "transpose");
  const float* ap = e.fptr(a, C * P, "transpose src");
  float* cp = e.fptr(c, C * P, "transpose out");
  if (!dry) launch_transpose(ap, cp, 1, (int)C, (int)P, scale, e.stream);
}

// engine/shaders/gn.comp:1-8: x [G][Cpg*S], gamma/beta [G*Cpg]
void op_group_norm(Engine& e, bool dry, long long x, long long g, long long b, long long out, long long G,
                   long long Cpg, long long S, float eps) {
  RVC_CHECK(G >= 0 && Cpg >= 1 && S >= 1, "group_norm: invalid shape");
  check_i32(Cpg, "group_norm");
  const float* xp = e.fptr(x, G * Cpg * S, "group_norm x");
  const float* gp = e.fptr(g, G * Cpg, "group_norm gamma");
  const float* bp = e.fptr(b, G * Cpg, "group_norm beta");
  float* op = e.fptr(out, G * Cpg * S, "group_norm out");
  if (!dry) launch_groupnorm_groups(xp, gp, bp, op, G, (int)Cpg, S, eps, e.stream);
}

// batch ops 12/16 (scores) and 13/17 (context); `used` 0 = the plain forms
void op_attn(Engine& e, bool dry, bool scores, long long a, long long b, long long used, long long out, long long H,
             long long T, long long D, long long C) {
  const char* nm = scores ? "attn_qk" : "attn_sv";
  RVC_CHECK(H >= 1 && T >= 1 && D >= 1 && H * D <= C, std::string(nm) + ": need H, T, D >= 1 and H*D <= C");
  check_i32(T, nm); check_i32(C, nm); check_i32(H, nm);
  const float* ap = e.fptr(a, scores ? T * C : H * T * T, nm);
  const float* bp = e.fptr(b, T * C, nm);
  const float* up = used ? e.fptr(used, (2 * T - 1) * D, nm) : nullptr;
  float* op = e.fptr(out, scores ? H * T * T : T * C, nm);
  if (dry) return;
  if (scores)
    launch_attn_scores(ap, bp, up, op, (int)H, (int)T, (int)D, (int)C, e.stream);
  else
    launch_attn_context(ap, bp, up, op, (int)H, (int)T, (int)D, (int)C, e.stream);
}

// Internal codes of the segment records (the reference records them as
// sub-view variants of ops 7/3/4/6/10/2/5).
enum SegOp : int {
  SEG_COPY = 100,
  SEG_ADD = 101,
  SEG_MUL = 102,
  SEG_LEAKY = 103,
  SEG_GELU = 104,
  SEG_CONV1D = 105,
  SEG_CONV_T1D = 106,
  REC_CONV2D = 110,    // rvc_batch_add_conv2d
  REC_CONV_T2D = 111,  // rvc_batch_add_conv_t2d
  REC_GRU = 112,       // rvc_batch_add_gru
};

const char* kBatchCodes =
    " (supported: 1 matmul 2 conv1d 3 add_inplace 4 mul_inplace 5 conv_t1d 6 leaky_relu 7 copy 8 softmax"
    " 9 layer_norm 10 gelu 11 bias_add 12 attn_qk 13 attn_sv 14 relu 15 group_norm 16 banded_attn_qk"
    " 17 banded_attn_sv 18 gating 19 transpose)";

bool public_code(int op) { return (op >= 1 && op <= 19); }

// ---- RMVPE ops (2-D conv, transposed 2-D conv, BiGRU): checked when recorded
// (dry), launched at commit or by the single-op exports

// engine/src/engine.zig:1602-1660 (see rvc_conv2d)
void op_conv2d(Engine& e, bool dry, long long x, long long w, long long b, long long out, long long B,
               long long c_in, long long H, long long W, long long c_out, long long kh, long long kw,
               long long pad_h, long long pad_w, long long stride_h, long long stride_w) {
  RVC_CHECK(B >= 1 && c_in >= 1 && H >= 1 && W >= 1 && c_out >= 1 && kh >= 1 && kw >= 1 && pad_h >= 0 &&
                pad_w >= 0 && stride_h >= 1 && stride_w >= 1,
            "conv2d: invalid dimensions");
  RVC_CHECK(kh <= H + 2 * pad_h && kw <= W + 2 * pad_w, "conv2d: kernel must fit the padded extent");
  RVC_CHECK(kh <= 3 && kw <= 3 && stride_h == stride_w && stride_h <= 2,
            "conv2d: this backend takes kernels up to 3x3 and one stride of 1 or 2 on both axes");
  RVC_CHECK(B * c_in * H * W < (1LL << 40) && c_in <= (1 << 20) && c_out <= (1 << 20), "conv2d: too large");
  const long long OH = (H + 2 * pad_h - kh) / stride_h + 1, OW = (W + 2 * pad_w - kw) / stride_w + 1;
  const float* xp = e.fptr(x, B * c_in * H * W, "conv2d x");
  const float* wp = e.fptr(w, c_out * c_in * kh * kw, "conv2d w");
  const float* bp = b ? e.fptr(b, c_out, "conv2d b") : nullptr;
  float* op = e.fptr(out, B * c_out * OH * OW, "conv2d out");
  if (dry) return;
  Conv2dLaunch a{};
  a.n_groups = 1;
  Conv2dGroup& g = a.g[0];
  g.ntaps = (int)(kh * kw);
  for (int i = 0; i < kh; ++i)
    for (int j = 0; j < kw; ++j) {
      g.dh[i * kw + j] = i - (int)pad_h;
      g.dw[i * kw + j] = j - (int)pad_w;
    }
  g.a_lim = g.oh_n = (int)OH;
  g.b_lim = g.ow_n = (int)OW;
  a.x = xp; a.xb = c_in * H * W; a.xc = H * W; a.H = (int)H; a.W = (int)W;
  a.out = op; a.ob = c_out * OH * OW; a.oc = OH * OW; a.ors = OW; a.ocs = 1;
  a.bias = bp; a.C_in = (int)c_in; a.C_out = (int)c_out; a.w_ld = packed_ld((int)c_out); a.B = (int)B;
  a.OH = (int)OH; a.OW = (int)OW; a.osh = a.osw = 1; a.stride = (int)stride_h;
  const size_t wfl = (size_t)kh * kw * c_in * a.w_ld;
  const size_t need = conv2d_split_floats(a);
  float* sc = static_cast<float*>(e.scratch_for(sizeof(float) * (wfl + need)));
  g.w = sc;
  if (need > 0) {
    a.part = sc + wfl;
    a.part_floats = need;
  }
  launch_pack_conv2d_weight(wp, sc, (int)c_out, (int)c_in, (int)kh, (int)kw, e.stream);
  launch_conv2d(a, e.stream);
}

// engine/src/engine.zig:1511-1560 (see rvc_conv_t2d); b == 0: no bias
void op_conv_t2d(Engine& e, bool dry, long long x, long long w, long long b, long long out, long long B,
                 long long c_in, long long ih, long long iw, long long c_out, long long kh, long long kw, long long sh,
                 long long sw, long long ph, long long pw, long long opad_h, long long opad_w, long long h_out,
                 long long w_out) {
  RVC_CHECK(B >= 1 && c_in >= 1 && ih >= 1 && iw >= 1 && c_out >= 1 && kh >= 1 && kw >= 1 && sh >= 1 && sw >= 1 &&
                ph >= 0 && pw >= 0 && opad_h >= 0 && opad_w >= 0,
            "conv_t2d: invalid dimensions");
  RVC_CHECK(opad_h < sh && opad_w < sw, "conv_t2d: output padding must be smaller than the stride");
  const long long hext = (ih - 1) * sh + (kh - 1), wext = (iw - 1) * sw + (kw - 1);
  RVC_CHECK(2 * ph <= hext && 2 * pw <= wext, "conv_t2d: padding must fit the upsampled extent");
  RVC_CHECK(h_out == hext + opad_h + 1 - 2 * ph && w_out == wext + opad_w + 1 - 2 * pw,
            "conv_t2d: h_out / w_out do not match the transposed-conv formula");
  RVC_CHECK(kh <= 3 && kw <= 3 && sh <= 2 && sw <= 2, "conv_t2d: this backend takes kernels up to 3x3 and strides up to 2");
  RVC_CHECK(B * c_in * ih * iw < (1LL << 40) && c_in <= (1 << 20) && c_out <= (1 << 20) && h_out * w_out < (1LL << 31),
            "conv_t2d: too large");
  const float* xp = e.fptr(x, B * c_in * ih * iw, "conv_t2d x");
  const float* wp = e.fptr(w, c_in * c_out * kh * kw, "conv_t2d w");
  const float* bp = b ? e.fptr(b, c_out, "conv_t2d b") : nullptr;
  float* op = e.fptr(out, B * c_out * h_out * w_out, "conv_t2d out");
  if (dry) return;
  Conv2dLaunch a{};
  ConvT2dTaps taps[kConv2dGroupsMax];
  int maxh = 0, maxw = 0;
  for (int c = 0; c < sh; ++c)
    for (int d = 0; d < sw; ++d) {
      const int oh_n = c < h_out ? (int)((h_out - c + sh - 1) / sh) : 0;
      const int ow_n = d < w_out ? (int)((w_out - d + sw - 1) / sw) : 0;
      if (oh_n == 0 || ow_n == 0) continue;
      Conv2dGroup& g = a.g[a.n_groups];
      ConvT2dTaps& t = taps[a.n_groups];
      t.n = 0;
      for (int i = 0; i < kh; ++i) {
        if ((c + ph - i) % sh != 0) continue;
        for (int j = 0; j < kw; ++j) {
          if ((d + pw - j) % sw != 0) continue;
          t.kh[t.n] = i;
          t.kw[t.n] = j;
          g.dh[t.n] = (int)((c + ph - i) / sh);
          g.dw[t.n] = (int)((d + pw - j) / sw);
          ++t.n;
        }
      }
      if (t.n == 0) {  // no tap reaches this phase: bias only
        t.n = 1;
        t.kh[0] = t.kw[0] = -1;
        g.dh[0] = g.dw[0] = 0;
      }
      g.ntaps = t.n;
      g.oh0 = c;
      g.ow0 = d;
      g.a_lim = g.oh_n = oh_n;
      g.b_lim = g.ow_n = ow_n;
      maxh = std::max(maxh, oh_n);
      maxw = std::max(maxw, ow_n);
      ++a.n_groups;
    }
  a.x = xp; a.xb = c_in * ih * iw; a.xc = ih * iw; a.H = (int)ih; a.W = (int)iw;
  a.out = op; a.ob = c_out * h_out * w_out; a.oc = h_out * w_out; a.ors = w_out; a.ocs = 1;
  a.bias = bp; a.C_in = (int)c_in; a.C_out = (int)c_out; a.w_ld = packed_ld((int)c_out); a.B = (int)B;
  a.OH = maxh; a.OW = maxw; a.osh = (int)sh; a.osw = (int)sw; a.stride = 1;
  size_t wfl = 0;
  for (int gi = 0; gi < a.n_groups; ++gi) wfl += (size_t)taps[gi].n * c_in * a.w_ld;
  const size_t need = conv2d_split_floats(a);
  float* sc = static_cast<float*>(e.scratch_for(sizeof(float) * (wfl + need)));
  size_t off = 0;
  for (int gi = 0; gi < a.n_groups; ++gi) {
    a.g[gi].w = sc + off;
    launch_pack_convt2d_phase(wp, sc + off, (int)c_in, (int)c_out, (int)kh, (int)kw, taps[gi], e.stream);
    off += (size_t)taps[gi].n * c_in * a.w_ld;
  }
  if (need > 0) {
    a.part = sc + wfl;
    a.part_floats = need;
  }
  launch_conv2d(a, e.stream);
}

// engine/src/engine.zig:3097-3112 (see rvc_gru); the error flag is checked
// after the next synchronisation (check_gru)
void op_gru(Engine& e, bool dry, long long a_, long long b_, long long c_, long long out, long long t,
            long long hdim) {
  RVC_CHECK(t >= 1 && hdim >= 1 && hdim <= 256 && t < (1LL << 30), "gru: need T >= 1 and 1 <= H <= 256");
  const long long k = 3 * hdim;
  GruArgs g{};
  g.gx = e.fptr(a_, 2 * t * k, "gru gx");
  g.whh = e.fptr(b_, 2 * k * hdim, "gru w_hh");
  g.bhh = e.fptr(c_, 2 * k, "gru b_hh");
  g.out = e.fptr(out, t * 2 * hdim, "gru out");
  if (dry) return;
  g.g_d = t * k; g.g_t = k; g.g_r = 1;
  g.o_d = hdim; g.o_t = 2 * hdim; g.o_j = 1;
  g.T = (int)t; g.H = (int)hdim; g.spin_limit = 1LL << 22;
  if (!e.gru_state) {
    void* p = nullptr;
    RVC_HIP(hipMalloc(&p, sizeof(unsigned long long) * (2 * 2 * 256 + 2)));
    e.gru_state = static_cast<unsigned long long*>(p);
  }
  g.state = e.gru_state;
  g.sync = reinterpret_cast<unsigned*>(e.gru_state + 2 * 2 * 256);
  // the error flag is sticky until check_gru reads it: the first GRU since
  // the last check clears it, later ones of the same batch keep a timeout
  // an earlier one reported
  g.keep_err = e.gru_pending ? 1 : 0;
  launch_bigru(g, e.stream);
  e.gru_pending = true;
}

// After a synchronisation: report a GRU launch whose step barrier gave up.
void check_gru(Engine& e) {
  if (!e.gru_pending) return;
  e.gru_pending = false;
  unsigned flag = 0;
  RVC_HIP(hipMemcpy(&flag, reinterpret_cast<unsigned*>(e.gru_state + 2 * 2 * 256) + 2, sizeof(unsigned),
                    hipMemcpyDeviceToHost));
  RVC_CHECK(flag == 0, "gru: step barrier timed out (workgroups not co-resident)");
}

void run_batch_op(Engine& e, const BatchOp& o, bool dry) {
  const long long* p = o.p;
  switch (o.op) {
    case 1: op_matmul(e, dry, o.a, o.b, o.c, p[0], p[1], p[2]); break;
    case REC_CONV2D:
      op_conv2d(e, dry, o.a, o.b, o.c, p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7], p[8], p[9], p[10], p[11]);
      break;
    case REC_CONV_T2D:
      op_conv_t2d(e, dry, o.a, o.b, o.c, p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7], p[8], p[9], p[10], p[11],
                  p[12], p[13], p[14], p[15]);
      break;
    case REC_GRU: op_gru(e, dry, o.a, o.b, o.c, p[0], p[1], p[2]); break;
    case 2: op_conv1d(e, dry, o.a, o.b, o.c, p[9], p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7], p[8]); break;
    case 3:
    case 4: {
      RVC_CHECK(p[0] >= 0, "add/mul_inplace: invalid size");
      float* ap = e.fptr(o.a, p[0], "inplace a");
      const float* bp = e.fptr(o.b, p[0], "inplace b");
      if (!dry) (o.op == 3 ? launch_add_inplace : launch_mul_inplace)(ap, bp, p[0], e.stream);
      break;
    }
    case 5: op_conv_t1d(e, dry, o.a, o.b, o.c, p[9], p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7], p[8]); break;
    case 6: {
      RVC_CHECK(p[0] >= 0, "leaky_relu: invalid size");
      float* ap = e.fptr(o.a, p[0], "leaky_relu a");
      if (!dry) launch_leaky(ap, p[0], bits_to_f32(p[1]), e.stream);
      break;
    }
    case 7: {
      RVC_CHECK(p[0] >= 0, "copy: invalid size");
      float* d = e.fptr(o.a, p[0], "copy dst");
      const float* s2 = e.fptr(o.b, p[0], "copy src");
      if (!dry) launch_copy(d, s2, p[0], e.stream);
      break;
    }
    case 8: op_softmax(e, dry, o.a, o.c, p[0], p[1]); break;
    case 9: op_layernorm(e, dry, o.a, o.b, o.c, p[9], p[0], p[1], bits_to_f32(p[2])); break;
    case 10: {
      RVC_CHECK(p[0] >= 0, "gelu: invalid size");
      float* ap = e.fptr(o.a, p[0], "gelu a");
      if (!dry) launch_gelu(ap, p[0], e.stream);
      break;
    }
    case 11: {
      RVC_CHECK(p[0] >= 0 && p[1] >= 1, "bias_add: need n >= 0 and cols >= 1");
      const float* ap = e.fptr(o.a, p[0], "bias_add a");
      const float* bp = e.fptr(o.b, p[1], "bias_add bias");
      float* cp = e.fptr(o.c, p[0], "bias_add out");
      if (!dry) launch_bias_add(cp, ap, bp, p[0], p[1], e.stream);
      break;
    }
    case 12: op_attn(e, dry, true, o.a, o.b, 0, o.c, p[0], p[1], p[2], p[3]); break;
    case 13: op_attn(e, dry, false, o.a, o.b, 0, o.c, p[0], p[1], p[2], p[3]); break;
    case 14: {
      RVC_CHECK(p[0] >= 0, "relu: invalid size");
      float* ap = e.fptr(o.a, p[0], "relu a");
      if (!dry) launch_relu(ap, p[0], e.stream);
      break;
    }
    case 15: op_group_norm(e, dry, o.a, o.b, o.c, p[9], p[0], p[1], p[2], bits_to_f32(p[3])); break;
    case 16:
      RVC_CHECK(o.c != 0, "banded_attn_qk: the relative table (c) is required");
      op_attn(e, dry, true, o.a, o.b, o.c, p[9], p[0], p[1], p[2], p[3]);
      break;
    case 17:
      RVC_CHECK(o.c != 0, "banded_attn_sv: the relative table (c) is required");
      op_attn(e, dry, false, o.a, o.b, o.c, p[9], p[0], p[1], p[2], p[3]);
      break;
    case 18: op_gating(e, dry, o.a, o.b, o.c, p[0], p[1], p[2], p[3]); break;
    case 19: op_transpose(e, dry, o.a, o.c, p[0], p[1], bits_to_f32(p[2])); break;
    case SEG_COPY:
    case SEG_ADD:
    case SEG_MUL: {  // a[a_off..+n) (=, +=, *=) b[b_off..+n)
      float* d = fview(e, o.a, p[1], p[0], "seg a");
      const float* s2 = fview(e, o.b, p[2], p[0], "seg b");
      if (dry) break;
      if (o.op == SEG_COPY) launch_copy(d, s2, p[0], e.stream);
      else if (o.op == SEG_ADD) launch_add_inplace(d, s2, p[0], e.stream);
      else launch_mul_inplace(d, s2, p[0], e.stream);
      break;
    }
    case SEG_LEAKY:
    case SEG_GELU: {  // a[a_off..+n) = act(a)
      float* d = fview(e, o.a, p[1], p[0], "seg a");
      if (dry) break;
      if (o.op == SEG_LEAKY) launch_leaky(d, p[0], bits_to_f32(p[2]), e.stream);
      else launch_gelu(d, p[0], e.stream);
      break;
    }
    case SEG_CONV1D:
      op_conv1d_seg(e, dry, o.a, o.b, o.c, p[9], p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7], p[8], p[10], p[11],
                    p[12]);
      break;
    case SEG_CONV_T1D: {
      long long q[22] = {o.a, o.b, o.c};
      for (int i = 0; i < 19; ++i) q[3 + i] = p[i];
      op_conv_t1d_seg(e, dry, q);
      break;
    }
    default: throw Error("invalid batch op code " + std::to_string(o.op) + kBatchCodes);
  }
}

}  // namespace

}  // namespace rvc

using namespace rvc;

// Run `body` under the engine's lock, translating exceptions to -1 + message.
template <class F>
static int32_t guarded(int64_t h, F&& body) {
  Engine* e = engine_from_handle(h);
  if (!e) {
    set_last_error("invalid engine handle");
    return -1;
  }
  try {
    std::lock_guard<std::mutex> lk(e->mu);
    body(*e);
    return 0;
  } catch (const std::exception& ex) {
    set_last_error(ex.what());
    return -1;
  }
}

extern "C" {

int64_t rvc_engine_create(void) {
  try {
    Engine* e = new Engine();
    std::lock_guard<std::mutex> lk(g_tab_mu);
    const long long h = g_next_handle++;
    g_engines[h] = e;
    g_last_engine = h;
    return h;
  } catch (const std::exception& ex) {
    set_last_error(ex.what());
    return -1;
  }
}

int32_t rvc_engine_destroy(int64_t h) {
  Engine* e = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_tab_mu);
    auto it = g_engines.find(h);
    if (it == g_engines.end()) {
      set_last_error("invalid engine handle");
      return -1;
    }
    e = it->second;
    g_engines.erase(it);
    if (g_last_engine == h) g_last_engine = 0;
  }
  { std::lock_guard<std::mutex> lk(e->mu); }
  delete e;
  return 0;
}

int32_t rvc_mem_upload(int64_t h, const float* src, int64_t n, int64_t* out_buf) {
  return rvc_mem_upload_bytes(h, src, n < 0 ? -1 : n * (int64_t)sizeof(float), out_buf);
}

int32_t rvc_mem_upload_bytes(int64_t h, const void* src, int64_t nbytes, int64_t* out_buf) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(nbytes >= 0 && out_buf, "mem_upload: invalid size");
    void* p = nullptr;
    RVC_HIP(hipMalloc(&p, nbytes > 0 ? (size_t)nbytes : 4));
    if (nbytes > 0) {
      hipError_t er = hipMemcpyAsync(p, src, (size_t)nbytes, hipMemcpyHostToDevice, e.stream);
      if (er == hipSuccess) er = hipStreamSynchronize(e.stream);
      if (er != hipSuccess) {
        (void)hipFree(p);
        throw Error(std::string("mem_upload: ") + hipGetErrorString(er));
      }
    }
    *out_buf = e.add_buffer(p, (size_t)(nbytes > 0 ? nbytes : 4));
  });
}

int32_t rvc_mem_upload_to(int64_t h, const float* src, int64_t n, int64_t buf) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(n >= 0, "mem_upload_to: invalid size");
    float* d = e.fptr(buf, n, "mem_upload_to");
    RVC_HIP(hipMemcpyAsync(d, src, (size_t)n * sizeof(float), hipMemcpyHostToDevice, e.stream));
    RVC_HIP(hipStreamSynchronize(e.stream));
  });
}

int32_t rvc_mem_alloc(int64_t h, int64_t nbytes, int64_t* out_buf) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(nbytes > 0 && out_buf, "mem_alloc: size must be > 0");
    void* p = nullptr;
    RVC_HIP(hipMalloc(&p, (size_t)nbytes));
    *out_buf = e.add_buffer(p, (size_t)nbytes);
  });
}

int32_t rvc_mem_fill_zero(int64_t h, int64_t buf, int64_t nbytes) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(nbytes > 0, "mem_fill_zero: size must be > 0");
    DevBuf& b = e.get(buf);
    RVC_CHECK((size_t)nbytes <= b.bytes, "mem_fill_zero: size exceeds buffer");
    // A fill kernel rather than a memset node keeps the stream capturable.
    RVC_CHECK(nbytes % 4 == 0, "mem_fill_zero: size must be a multiple of 4");
    launch_fill(static_cast<float*>(b.ptr), nbytes / 4, 0.f, e.stream);
  });
}

int32_t rvc_mem_download(int64_t h, int64_t buf, float* dst, int64_t n) {
  return rvc_mem_download_bytes(h, buf, dst, n < 0 ? -1 : n * (int64_t)sizeof(float));
}

int32_t rvc_mem_download_bytes(int64_t h, int64_t buf, void* dst, int64_t nbytes) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(nbytes >= 0, "mem_download: invalid size");
    DevBuf& b = e.get(buf);
    RVC_CHECK((size_t)nbytes <= b.bytes, "mem_download: size exceeds buffer");
    if (nbytes == 0) return;
    RVC_HIP(hipMemcpyAsync(dst, b.ptr, (size_t)nbytes, hipMemcpyDeviceToHost, e.stream));
    RVC_HIP(hipStreamSynchronize(e.stream));
  });
}

int32_t rvc_mem_free(int64_t h, int64_t buf) {
  return guarded(h, [&](Engine& e) {
    DevBuf& b = e.get(buf);
    RVC_HIP(hipStreamSynchronize(e.stream));
    RVC_HIP(hipFree(b.ptr));
    e.bufs.erase(buf);
  });
}

int32_t rvc_mem_upload_to_batch(int64_t h, int64_t n, const int64_t* sizes, const float* const* datas,
                                const int64_t* ids) {
  if (n <= 0) return engine_from_handle(h) ? 0 : guarded(h, [](Engine&) {});
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(sizes && datas && ids, "mem_upload_to_batch: null array");
    std::vector<float*> dst((size_t)n);
    for (int64_t i = 0; i < n; ++i) {
      RVC_CHECK(sizes[i] >= 0, "mem_upload_to_batch: negative size");
      dst[i] = e.fptr(ids[i], sizes[i], "mem_upload_to_batch");
    }
    for (int64_t i = 0; i < n; ++i)
      if (sizes[i] > 0)
        RVC_HIP(hipMemcpyAsync(dst[i], datas[i], (size_t)sizes[i] * sizeof(float), hipMemcpyHostToDevice, e.stream));
    RVC_HIP(hipStreamSynchronize(e.stream));
  });
}

int32_t rvc_mem_download_batch(int64_t h, const int64_t* bufs, uint8_t* const* dsts, const int64_t* sizes,
                               int64_t count) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(count >= 0, "mem_download_batch: negative count");
    if (count == 0) return;
    RVC_CHECK(bufs && dsts && sizes, "mem_download_batch: null array");
    std::vector<const float*> src((size_t)count);
    for (int64_t i = 0; i < count; ++i) {
      RVC_CHECK(sizes[i] >= 0, "mem_download_batch: negative size");
      src[i] = e.fptr(bufs[i], sizes[i], "mem_download_batch");
    }
    for (int64_t i = 0; i < count; ++i)
      if (sizes[i] > 0)
        RVC_HIP(hipMemcpyAsync(dsts[i], src[i], (size_t)sizes[i] * sizeof(float), hipMemcpyDeviceToHost, e.stream));
    RVC_HIP(hipStreamSynchronize(e.stream));
  });
}

int32_t rvc_matmul(int64_t h, int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n) {
  return guarded(h, [&](Engine& e) { submit(e, [&] { op_matmul(e, false, a, b, c, m, k, n); }); });
}

int32_t rvc_add(int64_t h, int64_t a, int64_t b, int64_t c, int64_t n) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(n >= 0, "add: invalid size");
    float* cp = e.fptr(c, n, "add c");
    const float* ap = e.fptr(a, n, "add a");
    const float* bp = e.fptr(b, n, "add b");
    submit(e, [&] { launch_add(cp, ap, bp, n, e.stream); });
  });
}

int32_t rvc_mul(int64_t h, int64_t a, int64_t b, int64_t c, int64_t n) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(n >= 0, "mul: invalid size");
    float* cp = e.fptr(c, n, "mul c");
    const float* ap = e.fptr(a, n, "mul a");
    const float* bp = e.fptr(b, n, "mul b");
    submit(e, [&] { launch_mul(cp, ap, bp, n, e.stream); });
  });
}

// Single ops that have a batch twin run through it (same checks, same kernels).
static int32_t single(int64_t h, int op, int64_t a, int64_t b, int64_t c, std::initializer_list<long long> ps) {
  return guarded(h, [&](Engine& e) {
    BatchOp o{op, a, b, c, {}};
    int i = 0;
    for (long long v : ps) o.p[i++] = v;
    submit(e, [&] { run_batch_op(e, o, false); });
  });
}

int32_t rvc_relu(int64_t h, int64_t a, int64_t n) { return single(h, 14, a, 0, 0, {n}); }

int32_t rvc_conv1d(int64_t h, int64_t x, int64_t w, int64_t b, int64_t out, int64_t B, int64_t c_in, int64_t l,
                   int64_t c_out, int64_t k, int64_t stride, int64_t pad_l, int64_t pad_r, int64_t dil) {
  return single(h, 2, x, w, b, {B, c_in, l, c_out, k, stride, pad_l, pad_r, dil, out});
}

int32_t rvc_conv_t1d(int64_t h, int64_t x, int64_t w, int64_t b, int64_t out, int64_t B, int64_t c_in, int64_t l,
                     int64_t c_out, int64_t k, int64_t stride, int64_t padding, int64_t output_padding, int64_t dil) {
  return single(h, 5, x, w, b, {B, c_in, l, c_out, k, stride, padding, output_padding, dil, out});
}

int32_t rvc_conv1d_noalloc(int64_t h, int64_t x, int64_t w, int64_t b, int64_t out, int64_t B, int64_t c_in,
                           int64_t l, int64_t c_out, int64_t k, int64_t stride, int64_t pad_l, int64_t pad_r,
                           int64_t dil) {
  // rvc_conv1d's kernels with the packed weights in the device's fixed
  // scratch: no hipMalloc / hipFree, no event, no library allocation
  return guarded(h, [&](Engine& e) {
    float* fixed = noalloc_scratch(e.device);
    op_conv1d(e, true, x, w, b, out, B, c_in, l, c_out, k, stride, pad_l, pad_r, dil, false, fixed,
              kNoAllocScratchFloats);
    op_conv1d(e, false, x, w, b, out, B, c_in, l, c_out, k, stride, pad_l, pad_r, dil, false, fixed,
              kNoAllocScratchFloats);
  });
}

int32_t rvc_conv1d_bf16(int64_t h, int64_t x, int64_t w, int64_t b, int64_t out, int64_t B, int64_t c_in, int64_t l,
                        int64_t c_out, int64_t k, int64_t stride, int64_t pad_l, int64_t pad_r, int64_t dil) {
  return guarded(h, [&](Engine& e) {
    op_conv1d(e, true, x, w, b, out, B, c_in, l, c_out, k, stride, pad_l, pad_r, dil, true);
    submit(e, [&] { op_conv1d(e, false, x, w, b, out, B, c_in, l, c_out, k, stride, pad_l, pad_r, dil, true); });
  });
}

int32_t rvc_conv_t1d_bf16(int64_t h, int64_t x, int64_t w, int64_t b, int64_t out, int64_t B, int64_t c_in,
                          int64_t l, int64_t c_out, int64_t k, int64_t stride, int64_t padding,
                          int64_t output_padding, int64_t dil) {
  return guarded(h, [&](Engine& e) {
    op_conv_t1d(e, true, x, w, b, out, B, c_in, l, c_out, k, stride, padding, output_padding, dil, true);
    submit(e, [&] {
      op_conv_t1d(e, false, x, w, b, out, B, c_in, l, c_out, k, stride, padding, output_padding, dil, true);
    });
  });
}

int32_t rvc_embed(int64_t h, int64_t ids, int64_t table, int64_t out, int64_t n, int64_t table_rows,
                  int64_t emb_dim) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(n >= 0 && table_rows >= 1 && emb_dim >= 1, "embed: invalid shape");
    DevBuf& ib = e.get(ids);
    RVC_CHECK((size_t)n * sizeof(int32_t) <= ib.bytes, "embed: ids buffer too small");
    const float* tp = e.fptr(table, table_rows * emb_dim, "embed table");
    float* op = e.fptr(out, n * emb_dim, "embed out");
    submit(e, [&] {
      launch_embed_i32(static_cast<const int*>(ib.ptr), tp, op, n, (int)table_rows, (int)emb_dim, e.stream);
    });
  });
}

int32_t rvc_add_inplace(int64_t h, int64_t a, int64_t b, int64_t n) { return single(h, 3, a, b, 0, {n}); }

int32_t rvc_mul_inplace(int64_t h, int64_t a, int64_t b, int64_t n) { return single(h, 4, a, b, 0, {n}); }

int32_t rvc_leaky_relu(int64_t h, int64_t a, int64_t n, int64_t slope) { return single(h, 6, a, 0, 0, {n, slope}); }

int32_t rvc_copy(int64_t h, int64_t dst, int64_t src, int64_t n) {
  if (dst == src) {
    set_last_error("copy: dst and src must be distinct buffers");
    return -1;
  }
  return single(h, 7, dst, src, 0, {n});
}

int32_t rvc_layernorm(int64_t h, int64_t x, int64_t gamma, int64_t beta, int64_t out, int64_t rows, int64_t cols,
                      double eps) {
  return guarded(h, [&](Engine& e) {
    submit(e, [&] { op_layernorm(e, false, x, gamma, beta, out, rows, cols, (float)eps); });
  });
}

int32_t rvc_rmsnorm(int64_t h, int64_t x, int64_t gamma, int64_t out, int64_t rows, int64_t cols, double eps) {
  return guarded(h, [&](Engine& e) { submit(e, [&] { op_rmsnorm(e, false, x, gamma, out, rows, cols, (float)eps); }); });
}

int32_t rvc_softmax(int64_t h, int64_t x, int64_t out, int64_t rows, int64_t cols) {
  return single(h, 8, x, 0, out, {rows, cols});
}

int32_t rvc_batch_begin(int64_t h) {
  return guarded(h, [&](Engine& e) { e.batch.clear(); });
}

// Check a record now (no launch) and append it to the pending batch.
static int32_t record(int64_t h, const BatchOp& o) {
  return guarded(h, [&](Engine& e) {
    run_batch_op(e, o, true);
    e.batch.push_back(o);
  });
}

int32_t rvc_batch_add(int64_t h, int32_t op, int64_t a, int64_t b, int64_t c, int64_t p0, int64_t p1, int64_t p2,
                      int64_t p3, int64_t p4, int64_t p5, int64_t p6, int64_t p7, int64_t p8, int64_t p9,
                      int64_t p10) {
  if (!public_code(op)) {
    if (!engine_from_handle(h)) return guarded(h, [](Engine&) {});
    set_last_error("invalid batch op code " + std::to_string(op) + kBatchCodes);
    return -1;
  }
  return record(h, BatchOp{op, a, b, c, {p0, p1, p2, p3, p4, p5, p6, p7, p8, p9, p10}});
}

int32_t rvc_batch_add_copy_seg(int64_t h, int64_t a, int64_t b, int64_t n, int64_t a_off, int64_t b_off) {
  return record(h, BatchOp{SEG_COPY, a, b, 0, {n, a_off, b_off}});
}

int32_t rvc_batch_add_add_seg(int64_t h, int64_t a, int64_t b, int64_t n, int64_t a_off, int64_t b_off) {
  return record(h, BatchOp{SEG_ADD, a, b, 0, {n, a_off, b_off}});
}

int32_t rvc_batch_add_mul_seg(int64_t h, int64_t a, int64_t b, int64_t n, int64_t a_off, int64_t b_off) {
  return record(h, BatchOp{SEG_MUL, a, b, 0, {n, a_off, b_off}});
}

int32_t rvc_batch_add_leaky_seg(int64_t h, int64_t a, int64_t n, int64_t a_off, int64_t slope) {
  return record(h, BatchOp{SEG_LEAKY, a, 0, 0, {n, a_off, slope}});
}

int32_t rvc_batch_add_gelu_seg(int64_t h, int64_t a, int64_t n, int64_t a_off) {
  return record(h, BatchOp{SEG_GELU, a, 0, 0, {n, a_off}});
}

int32_t rvc_batch_add_conv1d_seg(int64_t h, int64_t a, int64_t b, int64_t c, int64_t p0, int64_t p1, int64_t p2,
                                 int64_t p3, int64_t p4, int64_t p5, int64_t p6, int64_t p7, int64_t p8, int64_t p9,
                                 int64_t seg_len, int64_t lo_off, int64_t l_out_full) {
  return record(h, BatchOp{SEG_CONV1D, a, b, c, {p0, p1, p2, p3, p4, p5, p6, p7, p8, p9, seg_len, lo_off, l_out_full}});
}

int32_t rvc_batch_add_conv_t1d_seg(int64_t h, int64_t a, int64_t b, int64_t c, int64_t p0, int64_t p1, int64_t p2,
                                   int64_t p3, int64_t p4, int64_t p5, int64_t p6, int64_t p7, int64_t p8,
                                   int64_t p9, int64_t l_out, int64_t l_in_seg, int64_t in_off, int64_t lo_off,
                                   int64_t l_out_full, int64_t vx, int64_t vw, int64_t vb, int64_t vo) {
  return record(h, BatchOp{SEG_CONV_T1D, a, b, c,
                           {p0, p1, p2, p3, p4, p5, p6, p7, p8, p9, l_out, l_in_seg, in_off, lo_off, l_out_full, vx,
                            vw, vb, vo}});
}

static void commit_batch(Engine& e) {
  std::vector<BatchOp> ops;
  ops.swap(e.batch);
  submit(e, [&] {
    for (const BatchOp& o : ops) run_batch_op(e, o, false);
  });
}

int32_t rvc_batch_commit(int64_t h) {
  return guarded(h, [&](Engine& e) {
    commit_batch(e);
    e.sync();
    e.in_flight = false;
    check_gru(e);
  });
}

int32_t rvc_batch_commit_async(int64_t h) {
  return guarded(h, [&](Engine& e) {
    commit_batch(e);
    e.in_flight = true;
  });
}

int32_t rvc_batch_wait(int64_t h) {
  return guarded(h, [&](Engine& e) {
    e.sync();
    e.in_flight = false;
    check_gru(e);
  });
}

int32_t rvc_batch_discard(int64_t h) {
  return guarded(h, [&](Engine& e) { e.batch.clear(); });
}

int32_t rvc_device_name(char* buf, int64_t buf_size) {
  if (!buf || buf_size <= 0) return -1;
  long long h;
  {
    std::lock_guard<std::mutex> lk(g_tab_mu);
    h = g_last_engine;
  }
  Engine* e = h ? engine_from_handle(h) : nullptr;
  if (!e) {
    set_last_error("no engine created");
    return -1;
  }
  const std::string& n = e->device_name;
  const size_t m = std::min((size_t)buf_size - 1, n.size());
  std::memcpy(buf, n.data(), m);
  buf[m] = 0;
  return 0;
}

int32_t rvc_last_error(char* buf, int64_t buf_size) {
  if (!buf || buf_size <= 0) return -1;
  std::lock_guard<std::mutex> lk(g_err_mu);
  const size_t m = std::min((size_t)buf_size - 1, g_err.size());
  std::memcpy(buf, g_err.data(), m);
  buf[m] = 0;
  return 0;
}

// ---------------------------------------------------------------- stats
int32_t rvc_ts_stats(int64_t h, int64_t* busy_ns_out, int64_t* submits_out) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(busy_ns_out && submits_out, "ts_stats: null output");
    if (e.ts_on) e.ts_collect();
    *busy_ns_out = e.ts_busy_ns;
    *submits_out = e.ts_submits;
  });
}

int32_t rvc_ts_reset(int64_t h) {
  return guarded(h, [&](Engine& e) {
    if (e.ts_on) e.ts_collect();
    e.ts_busy_ns = 0;
    e.ts_submits = 0;
  });
}

int32_t rvc_mem_stats(int64_t h, int64_t* sub_total, int64_t* sub_chunks, int64_t* sub_free_bytes,
                      int64_t* sub_free_blocks, int64_t* buf_count, int64_t* buf_bytes, int64_t* staging_up,
                      int64_t* staging_dn, int64_t* direct_bytes, int64_t* max_buf_bytes, int64_t* max_buf_sub) {
  return guarded(h, [&](Engine& e) {
    int64_t* outs[] = {sub_total,  sub_chunks, sub_free_bytes, sub_free_blocks, buf_count,  buf_bytes,
                       staging_up, staging_dn, direct_bytes,   max_buf_bytes,   max_buf_sub};
    for (int64_t* p : outs) RVC_CHECK(p != nullptr, "mem_stats: null output");
    long long total = 0, mx = 0;
    for (auto& kv : e.bufs) {
      total += (long long)kv.second.bytes;
      mx = std::max(mx, (long long)kv.second.bytes);
    }
    // every buffer is its own device allocation: no suballocator chunks, no
    // free lists, no persistent staging buffers
    *sub_total = *sub_chunks = *sub_free_bytes = *sub_free_blocks = 0;
    *buf_count = (int64_t)e.bufs.size();
    *buf_bytes = total;
    *staging_up = *staging_dn = 0;
    *direct_bytes = total + (long long)e.scratch_bytes;
    *max_buf_bytes = mx;
    *max_buf_sub = 0;
  });
}

int64_t rvc_mem_top(int64_t h, int64_t n, int64_t* out) {
  Engine* e = engine_from_handle(h);
  if (!e) {
    set_last_error("invalid engine handle");
    return -1;
  }
  if (n <= 0) return 0;
  if (!out) {
    set_last_error("mem_top: null output");
    return -1;
  }
  std::lock_guard<std::mutex> lk(e->mu);
  std::vector<std::pair<long long, long long>> v;  // (bytes, device address)
  v.reserve(e->bufs.size());
  for (auto& kv : e->bufs) v.push_back({(long long)kv.second.bytes, (long long)(uintptr_t)kv.second.ptr});
  std::sort(v.begin(), v.end(), [](const auto& x, const auto& y) { return x.first > y.first; });
  const int64_t cnt = std::min<int64_t>(n, (int64_t)v.size());
  for (int64_t i = 0; i < cnt; ++i) {
    out[3 * i] = v[i].first;
    out[3 * i + 1] = 0;  // not suballocated
    out[3 * i + 2] = v[i].second;
  }
  return cnt;
}

// The reference reports Vulkan feature flags; the HIP device has each
// capability they stand for (fp16 arithmetic, matrix-multiply hardware,
// 16-bit/8-bit shader types), followed by the ISA name.
int32_t rvc_probe_extensions(int64_t h, char* buf, int64_t buf_size) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(buf && buf_size > 0, "probe_extensions: invalid buffer");
    hipDeviceProp_t prop;
    RVC_HIP(hipGetDeviceProperties(&prop, e.device));
    const std::string s = std::string("shaderFloat16=1,VK_KHR_cooperative_matrix=1,VK_KHR_shader_float16_int8=1,arch=") +
                          prop.gcnArchName;
    RVC_CHECK((int64_t)s.size() < buf_size, "probe_extensions: buffer too small");
    std::memcpy(buf, s.c_str(), s.size() + 1);
  });
}

// ---------------------------------------------------------------- not provided
// 2-D convolutions, GRU, im2col and the f16 matmul serve the reference's
// RMVPE pitch model and training paths, outside the synthesis path this
// library accelerates; they fail with a message like any invalid call.
static int32_t not_provided(const char* name) {
  set_last_error(std::string(name) +
                 ": not provided by the HIP backend (2-D conv / GRU / im2col / f16 matmul serve the pitch model "
                 "and training paths, outside the synthesis path)");
  return -1;
}

int32_t rvc_matmul_f16(int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t) {
  return not_provided("rvc_matmul_f16");
}
// engine/src/ffi.zig:378-426 + engine.zig:1602-1660: out[B][C_out][OH][OW] =
// conv2d(x[B][C_in][H][W], w[C_out][C_in][KH][KW]) + b (b == 0: none), symmetric
// zero padding, dilation 1.  The MFMA kernel takes kernels up to 3x3 and one
// stride of 1 or 2 on both axes (RMVPE's 3x3 / 1x1 convs and the 2x2 stride-2
// pooling conv); other shapes are rejected with a message.
int32_t rvc_conv2d(int64_t h, int64_t x, int64_t w, int64_t b, int64_t out, int64_t B, int64_t c_in, int64_t H,
                   int64_t W, int64_t c_out, int64_t kh, int64_t kw, int64_t pad_h, int64_t pad_w, int64_t stride_h,
                   int64_t stride_w) {
  return guarded(h, [&](Engine& e) {
    op_conv2d(e, true, x, w, b, out, B, c_in, H, W, c_out, kh, kw, pad_h, pad_w, stride_h, stride_w);
    submit(e, [&] { op_conv2d(e, false, x, w, b, out, B, c_in, H, W, c_out, kh, kw, pad_h, pad_w, stride_h, stride_w); });
  });
}
// engine/src/ffi.zig:428-479 + engine.zig:1511-1560: out[B][C_out][h_out][w_out]
// = conv_transpose2d(x[B][C_in][ih][iw], w[C_in][C_out][kh][kw]), stride (sh, sw),
// padding (ph, pw), output padding (opad_h, opad_w) < stride, no bias.  Output
// row o = c + sh*a of stride phase c takes the taps k = c + ph (mod sh) of input
// row a + (c + ph - k) / sh (columns alike); every phase is one group of the
// conv2d MFMA kernel with its own extent.  Kernels up to 3x3 and strides up to
// 2 on this backend.
int32_t rvc_conv_t2d(int64_t h, int64_t x, int64_t w, int64_t out, int64_t B, int64_t c_in, int64_t ih, int64_t iw,
                     int64_t c_out, int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                     int64_t opad_h, int64_t opad_w, int64_t h_out, int64_t w_out) {
  return guarded(h, [&](Engine& e) {
    op_conv_t2d(e, true, x, w, 0, out, B, c_in, ih, iw, c_out, kh, kw, sh, sw, ph, pw, opad_h, opad_w, h_out, w_out);
    submit(e, [&] {
      op_conv_t2d(e, false, x, w, 0, out, B, c_in, ih, iw, c_out, kh, kw, sh, sw, ph, pw, opad_h, opad_w, h_out,
                  w_out);
    });
  });
}

// engine/src/ffi.zig:481-496 + engine.zig:1704-1722: out[C][2H-1][2W-1] holds
// x[C][H][W] at even rows and columns, zeros elsewhere (C = batch x channels).
int32_t rvc_insert_zeros_2x(int64_t h, int64_t x, int64_t out, int64_t c, int64_t h_, int64_t w) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(c >= 1 && h_ >= 1 && w >= 1, "insert_zeros_2x: invalid dimensions");
    RVC_CHECK(c * (2 * h_ - 1) * (2 * w - 1) < (1LL << 40) && h_ < (1 << 30) && w < (1 << 30), "insert_zeros_2x: too large");
    const float* xp = e.fptr(x, c * h_ * w, "insert_zeros_2x x");
    float* op = e.fptr(out, c * (2 * h_ - 1) * (2 * w - 1), "insert_zeros_2x out");
    submit(e, [&] { launch_insert_zeros_2x(xp, op, c, (int)h_, (int)w, e.stream); });
  });
}
// engine/src/ffi.zig:1196-1244: rvc_conv2d recorded into the pending batch
int32_t rvc_batch_add_conv2d(int64_t h, int64_t x, int64_t w, int64_t b, int64_t out, int64_t B, int64_t c_in,
                             int64_t ih, int64_t iw, int64_t c_out, int64_t kh, int64_t kw, int64_t pad_h,
                             int64_t pad_w, int64_t stride_h, int64_t stride_w) {
  return record(h, BatchOp{REC_CONV2D, x, w, b, {out, B, c_in, ih, iw, c_out, kh, kw, pad_h, pad_w, stride_h, stride_w}});
}
// engine/src/ffi.zig:1246-1302: rvc_conv_t2d with a bias (b == 0: none),
// recorded into the pending batch
int32_t rvc_batch_add_conv_t2d(int64_t h, int64_t x, int64_t w, int64_t b, int64_t out, int64_t B, int64_t c_in,
                               int64_t ih, int64_t iw, int64_t c_out, int64_t kh, int64_t kw, int64_t sh, int64_t sw,
                               int64_t ph, int64_t pw, int64_t opad_h, int64_t opad_w, int64_t h_out, int64_t w_out) {
  return record(h, BatchOp{REC_CONV_T2D, x, w, b,
                           {out, B, c_in, ih, iw, c_out, kh, kw, sh, sw, ph, pw, opad_h, opad_w, h_out, w_out}});
}
int32_t rvc_batch_add_im2col_1d(int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                                int64_t, int64_t) {
  return not_provided("rvc_batch_add_im2col_1d");
}
int32_t rvc_batch_add_im2col_2d(int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                                int64_t, int64_t, int64_t, int64_t, int64_t, int64_t) {
  return not_provided("rvc_batch_add_im2col_2d");
}
// engine/src/ffi.zig:1377-1392: rvc_gru recorded into the pending batch (its
// barrier flag is checked by rvc_batch_commit / rvc_batch_wait)
int32_t rvc_batch_add_gru(int64_t h, int64_t a, int64_t b, int64_t c, int64_t out, int64_t t, int64_t hdim) {
  return record(h, BatchOp{REC_GRU, a, b, c, {out, t, hdim}});
}
// engine/src/ffi.zig:1394-1409 + engine.zig:3097-3112: bidirectional GRU
// recurrence over precomputed gate inputs a [2T][3H] (rows 0..T-1 forward,
// T..2T-1 reverse, both in time order), weights b = W_hh [2][3H][H], c = b_hh
// [2][3H]; out [T][2H] (forward units first).  H <= 256 as in the reference.
int32_t rvc_gru(int64_t h, int64_t a, int64_t b, int64_t c, int64_t out, int64_t t, int64_t hdim) {
  return guarded(h, [&](Engine& e) {
    op_gru(e, true, a, b, c, out, t, hdim);
    submit(e, [&] { op_gru(e, false, a, b, c, out, t, hdim); });
    e.sync();
    check_gru(e);
  });
}
int32_t rvc_batch_add_gru_sync(int64_t, int64_t, int64_t, int64_t) { return not_provided("rvc_batch_add_gru_sync"); }

}  // extern "C"
