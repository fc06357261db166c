// The C ABI of the HIP backend: engine / memory / single-op / record-commit
// exports with the reference's names, argument meaning and error convention
// (engine/src/ffi.zig:1-1119): every export returns int32 0 on success and
// -1 on failure with the message in a process-global, mutex-protected
// buffer read by rvc_last_error; rvc_engine_create returns an int64 handle
// or -1; buffer ids are opaque int64 keys, 0 meaning "no bias"; sizes are
// float counts except rvc_mem_alloc / rvc_mem_fill_zero (bytes); f32
// scalars travel as IEEE bit patterns in int64 (slope, batch eps, scale).
// Every call on an engine is serialised by its mutex.
#include <cmath>
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
}

Engine::~Engine() {
  if (stream) (void)hipStreamSynchronize(stream);
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

// ---------------------------------------------------------------- ops
namespace {

float bits_to_f32(long long v) {
  const uint32_t u = (uint32_t)((unsigned long long)v & 0xffffffffULL);
  float f;
  std::memcpy(&f, &u, 4);
  return f;
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

void op_conv1d(Engine& e, long long x, long long w, long long b, long long out, long long B, long long C_in,
               long long L, long long C_out, long long K, long long stride, long long pad_l, long long pad_r,
               long long dil) {
  RVC_CHECK(B >= 1 && C_in >= 1 && C_out >= 1 && K >= 1 && stride >= 1 && dil >= 1 && pad_l >= 0 &&
                pad_r >= 0 && L >= 0,
            "conv1d: invalid parameters (stride/dilation>=1, padding>=0, K>=1)");
  const long long n_out = (L + pad_l + pad_r - dil * (K - 1) - 1) / stride + 1;
  RVC_CHECK(n_out >= 1, "conv1d: empty output");
  const float* xp = e.fptr(x, B * C_in * L, "conv1d x");
  const float* wp = e.fptr(w, C_out * C_in * K, "conv1d w");
  const float* bp = b ? e.fptr(b, C_out, "conv1d bias") : nullptr;
  float* op = e.fptr(out, B * C_out * n_out, "conv1d out");
  if ((stride == 1 || stride == 2) && conv1d_mfma_supported((int)K, (int)dil)) {
    float* packed = static_cast<float*>(e.scratch_for(sizeof(float) * packed_ld((int)C_out) * C_in * K));
    launch_pack_conv_weight(wp, packed, (int)C_out, (int)C_in, (int)K, e.stream);
    launch_conv1d_mfma(one_conv(xp, C_in, L, packed, bp, op, C_out, n_out, B, K, dil, pad_l, stride), e.stream);
  } else {
    DirectConvArgs a{};
    a.x = xp; a.xb = C_in * L; a.xc = L;
    a.w = wp; a.bias = bp;
    a.out = op; a.ob = C_out * n_out; a.oc = n_out;
    a.C_in = (int)C_in; a.C_out = (int)C_out; a.L_in = (int)L; a.n_out = (int)n_out;
    a.K = (int)K; a.stride = (int)stride; a.dil = (int)dil; a.in_off = (int)-pad_l;
    a.combine = COMB_STORE; a.div = 1.f; a.B = (int)B;
    launch_conv1d_direct(a, e.stream);
  }
}

}  // namespace

// Polyphase ConvTranspose1d on the MFMA kernel (dilation 1): output o with
// (o + padding) = m*stride + r only sees taps k = r + j*stride of input
// m - j, so phase r is a stride-1 conv over m with J_r taps whose outputs land
// at o = m*stride + r - padding.  All phases go into one grouped launch.
// Shared by the op-level export and the synthesis session.
void convt_polyphase(hipStream_t st, const float* x, long long xb, long long xc, const float* const* w_phases,
                     const float* bias, float* out, long long ob, long long oc, int B, int C_in, int C_out, int L,
                     int n_out, int K, int stride, int padding, int in_act, float in_slope, int combine) {
  RVC_CHECK(stride >= 1 && stride <= kMaxConvGroups, "conv_transpose1d: stride exceeds the grouped launch");
  ConvLaunch a{};
  a.xb = xb; a.xc = xc; a.ob = ob; a.oc = oc;
  a.C_in = C_in; a.C_out = C_out; a.w_ld = packed_ld(C_out); a.L_in = L; a.B = B;
  a.in_act = in_act; a.in_slope = in_slope; a.div = 1.f;
  for (int r = 0; r < stride; ++r) {
    const int J = convt_phase_taps(K, stride, r);
    // m range with 0 <= m*stride + r - padding < n_out
    const int lo = padding - r;
    const int m0 = lo <= 0 ? 0 : (lo + stride - 1) / stride;
    const int hi = n_out - 1 - r + padding;
    if (hi < 0) continue;
    const int m1 = hi / stride;
    if (m1 < m0) continue;
    ConvGroup& g = a.g[a.n_groups++];
    g.x = x; g.w = w_phases[r]; g.bias = bias; g.res = nullptr; g.out = out;
    g.K = J; g.dil = 1; g.in_off = m0 - (J > 0 ? J - 1 : 0);
    g.out_step = stride; g.out_off = m0 * stride + r - padding;
    g.n_out = m1 - m0 + 1; g.combine = combine;
  }
  if (a.n_groups > 0) launch_conv1d_mfma(a, st);
}

namespace {

void op_conv_t1d(Engine& e, long long x, long long w, long long b, long long out, long long B, long long C_in,
                 long long L, long long C_out, long long K, long long stride, long long padding, long long opad,
                 long long dil) {
  RVC_CHECK(B >= 1 && C_in >= 1 && C_out >= 1 && K >= 1 && stride >= 1 && dil >= 1 && padding >= 0 &&
                opad >= 0 && L >= 1,
            "conv_transpose1d: invalid parameters (stride/dilation>=1, padding/output_padding>=0)");
  const long long n_out = (L - 1) * stride - 2 * padding + dil * (K - 1) + opad + 1;
  RVC_CHECK(n_out >= 1, "conv_transpose1d: empty output");
  const float* xp = e.fptr(x, B * C_in * L, "conv_t1d x");
  const float* wp = e.fptr(w, C_in * C_out * K, "conv_t1d w");
  const float* bp = b ? e.fptr(b, C_out, "conv_t1d bias") : nullptr;
  float* op = e.fptr(out, B * C_out * n_out, "conv_t1d out");
  const int ld = packed_ld((int)C_out);
  if (dil == 1 && stride <= kMaxConvGroups && (K + stride - 1) / stride <= kConvTapsMax) {
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
    convt_polyphase(e.stream, xp, C_in * L, L, phases.data(), bp, op, C_out * n_out, n_out, (int)B, (int)C_in,
                    (int)C_out, (int)L, (int)n_out, (int)K, (int)stride, (int)padding, ACT_NONE, 0.f, COMB_STORE);
  } else {
    ConvTArgs a{};
    a.x = xp; a.xb = C_in * L; a.xc = L;
    a.w = wp; a.bias = bp;
    a.out = op; a.ob = C_out * n_out; a.oc = n_out;
    a.C_in = (int)C_in; a.C_out = (int)C_out; a.L_in = (int)L; a.n_out = (int)n_out;
    a.K = (int)K; a.stride = (int)stride; a.padding = (int)padding; a.dil = (int)dil;
    a.combine = COMB_STORE; a.B = (int)B;
    launch_conv_t1d_direct(a, e.stream);
  }
}

void op_matmul(Engine& e, long long a, long long b, long long c, long long M, long long K, long long N) {
  RVC_CHECK(M >= 1 && K >= 1 && N >= 1, "matmul: invalid shape");
  const float* ap = e.fptr(a, M * K, "matmul a");
  const float* bp = e.fptr(b, K * N, "matmul b");
  float* cp = e.fptr(c, M * N, "matmul c");
  // c[M][N] = a[M][K] b[K][N] as a 1x1 conv: channels = K, time = N; the
  // packed weights are a^T (a seen as a [M][K][1] conv weight).
  float* at = static_cast<float*>(e.scratch_for(sizeof(float) * packed_ld((int)M) * K));
  launch_pack_conv_weight(ap, at, (int)M, (int)K, 1, e.stream);
  launch_conv1d_mfma(one_conv(bp, K, N, at, nullptr, cp, M, N, 1, 1, 1, 0), e.stream);
}

void op_layernorm(Engine& e, long long x, long long g, long long b, long long out, long long rows, long long cols,
                  float eps) {
  RVC_CHECK(rows >= 0 && cols >= 1, "layer_norm: invalid shape");
  const float* xp = e.fptr(x, rows * cols, "layer_norm x");
  const float* gp = e.fptr(g, cols, "layer_norm gamma");
  const float* bp = e.fptr(b, cols, "layer_norm beta");
  float* op = e.fptr(out, rows * cols, "layer_norm out");
  launch_layernorm_rows(xp, gp, bp, op, rows, (int)cols, eps, e.stream);
}

void op_softmax(Engine& e, long long x, long long out, long long rows, long long cols) {
  RVC_CHECK(rows >= 0 && cols >= 1, "softmax: invalid shape");
  launch_softmax_rows(e.fptr(x, rows * cols, "softmax x"), e.fptr(out, rows * cols, "softmax out"), rows,
                      (int)cols, e.stream);
}

void op_gating(Engine& e, long long a, long long b, long long c, long long n, long long lg, long long h,
               long long off);

void op_transpose(Engine& e, long long a, long long c, long long C, long long P, float scale) {
  RVC_CHECK(C >= 1 && P >= 1, "transpose: invalid shape");
  launch_transpose(e.fptr(a, C * P, "transpose src"), e.fptr(c, C * P, "transpose out"), 1, (int)C, (int)P,
                   scale, e.stream);
}

void run_batch_op(Engine& e, const BatchOp& o) {
  const long long* p = o.p;
  switch (o.op) {
    case 1: op_matmul(e, o.a, o.b, o.c, p[0], p[1], p[2]); break;
    case 2: op_conv1d(e, o.a, o.b, o.c, p[9], p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7], p[8]); break;
    case 3: launch_add_inplace(e.fptr(o.a, p[0], "add_inplace a"), e.fptr(o.b, p[0], "add_inplace b"), p[0],
                               e.stream); break;
    case 4: launch_mul_inplace(e.fptr(o.a, p[0], "mul_inplace a"), e.fptr(o.b, p[0], "mul_inplace b"), p[0],
                               e.stream); break;
    case 5: op_conv_t1d(e, o.a, o.b, o.c, p[9], p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7], p[8]); break;
    case 6: launch_leaky(e.fptr(o.a, p[0], "leaky_relu a"), p[0], bits_to_f32(p[1]), e.stream); break;
    case 7: launch_copy(e.fptr(o.a, p[0], "copy dst"), e.fptr(o.b, p[0], "copy src"), p[0], e.stream); break;
    case 8: op_softmax(e, o.a, o.c, p[0], p[1]); break;
    case 9: op_layernorm(e, o.a, o.b, o.c, p[9], p[0], p[1], bits_to_f32(p[2])); break;
    case 14: launch_relu(e.fptr(o.a, p[0], "relu a"), p[0], e.stream); break;
    case 18: op_gating(e, o.a, o.b, o.c, p[0], p[1], p[2], p[3]); break;
    case 19: op_transpose(e, o.a, o.c, p[0], p[1], bits_to_f32(p[2])); break;
    case 100: {  // copy segment: dst[a_off..+n) = src[b_off..+n)
      float* d = e.fptr(o.a, p[1] + p[0], "copy_seg dst");
      const float* s2 = e.fptr(o.b, p[2] + p[0], "copy_seg src");
      launch_copy(d + p[1], s2 + p[2], p[0], e.stream);
      break;
    }
    default: throw Error("invalid batch op code " + std::to_string(o.op) +
                         " (supported: 1 matmul 2 conv1d 3 add_inplace 4 mul_inplace 5 conv_t1d 6 leaky_relu"
                         " 7 copy 8 softmax 9 layer_norm 14 relu 18 gating 19 transpose)");
  }
}

}  // namespace



namespace {
void op_gating(Engine& e, long long a, long long b, long long c, long long n, long long lg, long long h,
               long long off) {
  RVC_CHECK(n >= 1 && h >= 1 && n % h == 0 && (lg == 1 || lg == n / h) && off >= 0, "gating: invalid parameters");
  const float* ap = e.fptr(a, 2 * n, "gating a");
  const float* gp = e.fptr(b, off + 2 * h * lg, "gating g");
  float* cp = e.fptr(c, n, "gating out");
  launch_gating(ap, gp, cp, n, (int)lg, (int)h, off, e.stream);
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

int32_t rvc_matmul(int64_t h, int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n) {
  return guarded(h, [&](Engine& e) { op_matmul(e, a, b, c, m, k, n); });
}

int32_t rvc_add(int64_t h, int64_t a, int64_t b, int64_t c, int64_t n) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(n >= 0, "add: invalid size");
    launch_add(e.fptr(c, n, "add c"), e.fptr(a, n, "add a"), e.fptr(b, n, "add b"), n, e.stream);
  });
}

int32_t rvc_mul(int64_t h, int64_t a, int64_t b, int64_t c, int64_t n) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(n >= 0, "mul: invalid size");
    launch_mul(e.fptr(c, n, "mul c"), e.fptr(a, n, "mul a"), e.fptr(b, n, "mul b"), n, e.stream);
  });
}

int32_t rvc_relu(int64_t h, int64_t a, int64_t n) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(n >= 0, "relu: invalid size");
    launch_relu(e.fptr(a, n, "relu a"), n, e.stream);
  });
}

int32_t rvc_conv1d(int64_t h, int64_t x, int64_t w, int64_t b, int64_t out, int64_t B, int64_t c_in, int64_t l,
                   int64_t c_out, int64_t k, int64_t stride, int64_t pad_l, int64_t pad_r, int64_t dil) {
  return guarded(h, [&](Engine& e) { op_conv1d(e, x, w, b, out, B, c_in, l, c_out, k, stride, pad_l, pad_r, dil); });
}

int32_t rvc_conv_t1d(int64_t h, int64_t x, int64_t w, int64_t b, int64_t out, int64_t B, int64_t c_in, int64_t l,
                     int64_t c_out, int64_t k, int64_t stride, int64_t padding, int64_t output_padding, int64_t dil) {
  return guarded(h, [&](Engine& e) {
    op_conv_t1d(e, x, w, b, out, B, c_in, l, c_out, k, stride, padding, output_padding, dil);
  });
}

int32_t rvc_embed(int64_t h, int64_t ids, int64_t table, int64_t out, int64_t n, int64_t table_rows,
                  int64_t emb_dim) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(n >= 0 && table_rows >= 1 && emb_dim >= 1, "embed: invalid shape");
    DevBuf& ib = e.get(ids);
    RVC_CHECK((size_t)n * sizeof(int32_t) <= ib.bytes, "embed: ids buffer too small");
    launch_embed_i32(static_cast<const int*>(ib.ptr), e.fptr(table, table_rows * emb_dim, "embed table"),
                     e.fptr(out, n * emb_dim, "embed out"), n, (int)table_rows, (int)emb_dim, e.stream);
  });
}

int32_t rvc_add_inplace(int64_t h, int64_t a, int64_t b, int64_t n) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(n >= 0, "add_inplace: invalid size");
    launch_add_inplace(e.fptr(a, n, "add_inplace a"), e.fptr(b, n, "add_inplace b"), n, e.stream);
  });
}

int32_t rvc_mul_inplace(int64_t h, int64_t a, int64_t b, int64_t n) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(n >= 0, "mul_inplace: invalid size");
    launch_mul_inplace(e.fptr(a, n, "mul_inplace a"), e.fptr(b, n, "mul_inplace b"), n, e.stream);
  });
}

int32_t rvc_leaky_relu(int64_t h, int64_t a, int64_t n, int64_t slope) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(n >= 0, "leaky_relu: invalid size");
    launch_leaky(e.fptr(a, n, "leaky_relu a"), n, bits_to_f32(slope), e.stream);
  });
}

int32_t rvc_copy(int64_t h, int64_t dst, int64_t src, int64_t n) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(n >= 0, "copy: invalid size");
    RVC_CHECK(dst != src, "copy: dst and src must be distinct buffers");
    launch_copy(e.fptr(dst, n, "copy dst"), e.fptr(src, n, "copy src"), n, e.stream);
  });
}

int32_t rvc_layernorm(int64_t h, int64_t x, int64_t gamma, int64_t beta, int64_t out, int64_t rows, int64_t cols,
                      double eps) {
  return guarded(h, [&](Engine& e) { op_layernorm(e, x, gamma, beta, out, rows, cols, (float)eps); });
}

int32_t rvc_softmax(int64_t h, int64_t x, int64_t out, int64_t rows, int64_t cols) {
  return guarded(h, [&](Engine& e) { op_softmax(e, x, out, rows, cols); });
}

int32_t rvc_batch_begin(int64_t h) {
  return guarded(h, [&](Engine& e) { e.batch.clear(); });
}

int32_t rvc_batch_add(int64_t h, int32_t op, int64_t a, int64_t b, int64_t c, int64_t p0, int64_t p1, int64_t p2,
                      int64_t p3, int64_t p4, int64_t p5, int64_t p6, int64_t p7, int64_t p8, int64_t p9,
                      int64_t p10) {
  return guarded(h, [&](Engine& e) {
    static const int ok[] = {1, 2, 3, 4, 5, 6, 7, 8, 9, 14, 18, 19};
    bool valid = false;
    for (int v : ok) valid |= (v == op);
    if (!valid)
      throw Error("invalid batch op code " + std::to_string(op) +
                  " (supported: 1 matmul 2 conv1d 3 add_inplace 4 mul_inplace 5 conv_t1d 6 leaky_relu 7 copy"
                  " 8 softmax 9 layer_norm 14 relu 18 gating 19 transpose)");
    BatchOp o{op, a, b, c, {p0, p1, p2, p3, p4, p5, p6, p7, p8, p9, p10}};
    e.batch.push_back(o);
  });
}

int32_t rvc_batch_add_copy_seg(int64_t h, int64_t a, int64_t b, int64_t n, int64_t a_off, int64_t b_off) {
  return guarded(h, [&](Engine& e) {
    RVC_CHECK(n >= 0 && a_off >= 0 && b_off >= 0, "copy_seg: invalid parameters");
    BatchOp o{100, a, b, 0, {n, a_off, b_off, 0, 0, 0, 0, 0, 0, 0, 0}};
    e.batch.push_back(o);
  });
}

static void commit_batch(Engine& e) {
  std::vector<BatchOp> ops;
  ops.swap(e.batch);
  for (const BatchOp& o : ops) run_batch_op(e, o);
}

int32_t rvc_batch_commit(int64_t h) {
  return guarded(h, [&](Engine& e) {
    commit_batch(e);
    e.sync();
    e.in_flight = false;
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

}  // extern "C"
