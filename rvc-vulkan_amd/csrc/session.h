// Shared machinery of the device-resident sessions (rvc_synth_*, rvc_hubert_*):
// checkpoint tensors staged on the host by key until finalize, packed device
// weights owned by the session, a named workspace of device buffers reused
// across calls, and per-launch HIP-event timing selected by a tag prefix.
#pragma once

#include <algorithm>
#include <cstring>

#include "engine.h"

namespace rvc {

struct HostT {
  std::vector<float> data;
  std::vector<long long> shape;
};

struct SessionBase {
  Engine* eng = nullptr;
  std::map<std::string, HostT> host;
  bool ready = false;
  std::vector<void*> owned;
  std::map<std::string, std::pair<float*, size_t>> ws;

  // timing
  std::string tag;
  struct Ev {
    hipEvent_t a, b;
    double flops, bytes;
    long long n;  // launches between the two events
  };
  // Consecutive timed launches on one stream share one event pair: an event
  // record between two kernels costs several microseconds of idle GPU, which
  // would otherwise land inside the very region being timed.  The end event
  // b is attached to the span's kernels themselves where the launch site
  // supports it (stop_hook()); b_done: the span's last launch did so.
  struct Span {
    bool open = false;
    hipEvent_t a{}, b{};
    bool b_done = false;
    hipStream_t st{};
    double flops = 0, bytes = 0;
    long long n = 0;
  } span;
  int run_depth = 0;
  std::vector<Ev> pending;
  std::vector<hipEvent_t> pool;
  double t_ms = 0, t_flops = 0, t_bytes = 0;
  long long t_n = 0;

  virtual ~SessionBase() {
    if (eng && eng->stream) (void)hipStreamSynchronize(eng->stream);
    for (void* p : owned) (void)hipFree(p);
    for (auto& kv : ws) (void)hipFree(kv.second.first);
    if (span.open) pool.push_back(span.a), pool.push_back(span.b);
    for (auto& e : pending) pool.push_back(e.a), pool.push_back(e.b);
    for (hipEvent_t e : pool) (void)hipEventDestroy(e);
  }

  // -------------------------------------------------------------- host weights
  void set_weight(const char* key, const float* data, const int64_t* shape, int ndim) {
    RVC_CHECK(!ready, "session already finalized");
    RVC_CHECK(key && data && shape && ndim >= 1 && ndim <= 8, "set_weight: invalid arguments");
    HostT t;
    long long n = 1;
    for (int i = 0; i < ndim; ++i) {
      RVC_CHECK(shape[i] >= 0, "set_weight: negative dimension");
      t.shape.push_back(shape[i]);
      n *= shape[i];
    }
    t.data.assign(data, data + n);
    host[key] = std::move(t);
  }
  const HostT& W(const std::string& k) const {
    auto it = host.find(k);
    if (it == host.end()) throw Error("missing weight: " + k);
    return it->second;
  }
  bool has(const std::string& k) const { return host.count(k) != 0; }

  static void check_shape(const std::string& k, const std::vector<long long>& got, std::vector<long long> want) {
    if (got != want) {
      std::string g, wv;
      for (auto x : got) g += std::to_string(x) + ",";
      for (auto x : want) wv += std::to_string(x) + ",";
      throw Error("weight " + k + " has shape [" + g + "], expected [" + wv + "]");
    }
  }

  // [C_out][C_in][K] -> [K][C_in][packed_ld(C_out)], pad columns zero
  static std::vector<float> pack(const std::vector<float>& w, long long C_out, long long C_in, long long K) {
    const long long ld = packed_ld((int)C_out);
    std::vector<float> o((size_t)(K * C_in * ld), 0.f);
    for (long long co = 0; co < C_out; ++co)
      for (long long ci = 0; ci < C_in; ++ci)
        for (long long k = 0; k < K; ++k) o[(k * C_in + ci) * ld + co] = w[(co * C_in + ci) * K + k];
    return o;
  }

  // [O][K] (a 1x1 conv) -> the A operands of v_mfma_f32_16x16x4_f32 in load
  // order, for kernels that keep a 16-row block's weights in registers: block
  // b (rows 16 b ..), step group j (k in [16 j, 16 j + 16)), lane l = 16 q + r
  // holds float4 {W[16 b + r][16 j + 4 u + q], u = 0..3}, at
  // ((b * (K / 16) + j) * 64 + l) * 4 + u.  A wave's load of group j is then
  // 64 consecutive float4s.
  static std::vector<float> pack_mfma_lanes(const std::vector<float>& w, long long O, long long K) {
    RVC_CHECK(O % 16 == 0 && K % 16 == 0 && (long long)w.size() == O * K,
              "pack_mfma_lanes: O and K must be multiples of 16");
    std::vector<float> r(w.size());
    for (long long b = 0; b < O / 16; ++b)
      for (long long j = 0; j < K / 16; ++j)
        for (long long l = 0; l < 64; ++l)
          for (long long u = 0; u < 4; ++u)
            r[((b * (K / 16) + j) * 64 + l) * 4 + u] = w[(16 * b + l % 16) * K + 16 * j + 4 * u + l / 16];
    return r;
  }

  // [C_out][C_in][K] -> bf16 [K][C_out][bf16_ld(C_in)], pad channels zero
  static std::vector<uint16_t> pack_bf16(const std::vector<float>& w, long long C_out, long long C_in, long long K) {
    const long long ld = bf16_ld((int)C_in);
    std::vector<uint16_t> o((size_t)(K * C_out * ld), 0);
    for (long long co = 0; co < C_out; ++co)
      for (long long ci = 0; ci < C_in; ++ci)
        for (long long k = 0; k < K; ++k) o[(k * C_out + co) * ld + ci] = f32_to_bf16(w[(co * C_in + ci) * K + k]);
    return o;
  }

  uint16_t* upload16(const std::vector<uint16_t>& v) {
    void* p = nullptr;
    RVC_HIP(hipMalloc(&p, std::max<size_t>(v.size(), 8) * sizeof(uint16_t)));
    owned.push_back(p);
    if (!v.empty()) RVC_HIP(hipMemcpy(p, v.data(), v.size() * sizeof(uint16_t), hipMemcpyHostToDevice));
    return static_cast<uint16_t*>(p);
  }

  float* upload(const std::vector<float>& v) {
    void* p = nullptr;
    RVC_HIP(hipMalloc(&p, std::max<size_t>(v.size(), 1) * sizeof(float)));
    owned.push_back(p);
    if (!v.empty()) RVC_HIP(hipMemcpy(p, v.data(), v.size() * sizeof(float), hipMemcpyHostToDevice));
    return static_cast<float*>(p);
  }
  float* upload_key(const std::string& k) { return upload(W(k).data); }
  float* upload_vec(const std::string& k, long long n) {
    const HostT& t = W(k);
    RVC_CHECK((long long)t.data.size() == n, "weight " + k + " must hold " + std::to_string(n) + " values");
    return upload(t.data);
  }

  // item-queue counters of this session's persistent conv launches (all on
  // the engine stream, so one launch at a time uses them); zeroed once here,
  // then reset by each launch's last workgroup
  unsigned* pq = nullptr;
  unsigned* persist_queue() {
    if (!pq) {
      void* p = nullptr;
      RVC_HIP(hipMalloc(&p, 16 * sizeof(unsigned)));
      owned.push_back(p);
      RVC_HIP(hipMemsetAsync(p, 0, 16 * sizeof(unsigned), eng->stream));
      pq = static_cast<unsigned*>(p);
    }
    return pq;
  }

  // -------------------------------------------------------------- workspace
  float* buf(const std::string& name, size_t n) {
    auto it = ws.find(name);
    if (it != ws.end() && it->second.second >= n) return it->second.first;
    RVC_HIP(hipStreamSynchronize(eng->stream));
    if (it != ws.end()) {
      RVC_HIP(hipFree(it->second.first));
      ws.erase(it);
    }
    void* p = nullptr;
    RVC_HIP(hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(float)));
    ws[name] = {static_cast<float*>(p), n};
    return static_cast<float*>(p);
  }
  void read(const std::string& nm, float* dst, long long n) {
    auto it = ws.find(nm);
    RVC_CHECK(it != ws.end(), "read: no intermediate named " + nm);
    RVC_CHECK((size_t)n <= it->second.second, "read: " + nm + " holds fewer values");
    RVC_HIP(hipMemcpyAsync(dst, it->second.first, sizeof(float) * n, hipMemcpyDeviceToHost, eng->stream));
    RVC_HIP(hipStreamSynchronize(eng->stream));
  }

  // -------------------------------------------------------------- timing
  bool timed(const char* t) const { return !tag.empty() && std::strncmp(t, tag.c_str(), tag.size()) == 0; }
  hipEvent_t ev() {
    if (!pool.empty()) {
      hipEvent_t e = pool.back();
      pool.pop_back();
      return e;
    }
    hipEvent_t e;
    RVC_HIP(hipEventCreate(&e));
    return e;
  }
  // Run fn (launches on stream st, the engine stream by default).  A timed
  // tag joins the open span on that stream (or opens one with a start
  // event); an untimed launch, a launch on another stream or close_span()
  // ends the span with its end event.  Launches nested inside fn are part of
  // the outer one.
  template <class Fn>
  void run(const char* t, double flops, double bytes, Fn&& fn, hipStream_t st = nullptr) {
    if (run_depth > 0) {
      fn();
      return;
    }
    if (!st) st = eng->stream;
    struct Depth {  // also restored when fn throws
      int& d;
      explicit Depth(int& x) : d(x) { ++d; }
      ~Depth() { --d; }
    };
    if (!timed(t)) {
      close_span();
      Depth dg(run_depth);
      fn();
      return;
    }
    if (span.open && span.st != st) close_span();
    if (!span.open) {
      span = Span{};
      span.open = true;
      span.a = ev();
      span.b = ev();
      span.st = st;
      RVC_HIP(hipEventRecord(span.a, st));
    }
    span.b_done = false;  // until this launch attaches the end event (not if fn throws)
    {
      Depth dg(run_depth);
      struct Hook {  // the span's end event for launch_timed(), cleared also when fn throws
        StopHook& h;
        explicit Hook(StopHook& x, hipEvent_t e) : h(x) { h = StopHook{e, 0}; }
        ~Hook() { h = StopHook{}; }
      } hook(stop_hook(), span.b);
      fn();
      span.b_done = hook.h.used > 0;
    }
    span.flops += flops;
    span.bytes += bytes;
    ++span.n;
  }
  // Ends the open span; sessions call it after their last launch and before
  // the copies and synchronisation that end a call.
  void close_span() {
    if (!span.open) return;
    span.open = false;
    if (!span.b_done) RVC_HIP(hipEventRecord(span.b, span.st));
    pending.push_back(Ev{span.a, span.b, span.flops, span.bytes, span.n});
  }
  void collect_timing() {
    // Only a call that ended early (an error) leaves a span open here; its
    // end event then lands after the synchronisation.
    close_span();
    for (auto& e : pending) {
      float ms = 0;
      RVC_HIP(hipEventElapsedTime(&ms, e.a, e.b));
      t_ms += ms;
      t_flops += e.flops;
      t_bytes += e.bytes;
      t_n += e.n;
      pool.push_back(e.a);
      pool.push_back(e.b);
    }
    pending.clear();
  }
  void set_timing(const char* t) {
    if (span.open) pool.push_back(span.a), pool.push_back(span.b);
    span.open = false;
    tag = t ? t : "";
    t_ms = t_flops = t_bytes = 0;
    t_n = 0;
  }

  // -------------------------------------------------------------- conv helpers
  // One conv x [B][C_in][L_in] -> out [B][C_out][n_out]: output i reads
  // x[i*stride - pad + k*dil].
  static ConvLaunch cargs(const float* x, long long xb, long long xc, const float* w, const float* bias, float* out,
                          long long ob, long long oc, int B, int C_in, int C_out, int L_in, int n_out, int K, int dil,
                          int pad, int stride = 1) {
    ConvLaunch a{};
    a.n_groups = 1;
    ConvGroup& g = a.g[0];
    g.x = x; g.w = w; g.bias = bias; g.res = nullptr; g.out = out;
    g.K = K; g.dil = dil; g.in_off = -pad; g.in_step = stride; g.out_step = 1; g.out_off = 0; g.n_out = n_out;
    g.combine = COMB_STORE;
    a.xb = xb; a.xc = xc; a.ob = ob; a.oc = oc;
    a.C_in = C_in; a.C_out = C_out; a.w_ld = packed_ld(C_out); a.L_in = L_in; a.B = B;
    a.div = 1.f;
    return a;
  }
  // stride-1 conv with output length == input length L ("same" padding)
  static ConvLaunch cargs_same(const float* x, long long xb, long long xc, const float* w, const float* bias,
                               float* out, long long ob, long long oc, int B, int C_in, int C_out, int L, int K,
                               int dil, int pad) {
    return cargs(x, xb, xc, w, bias, out, ob, oc, B, C_in, C_out, L, L, K, dil, pad);
  }
  // 1x1 conv: x [B][C_in][L] -> out [B][C_out][L]
  static ConvLaunch c1x1(const float* x, long long xb, const float* w, const float* b, float* out, int B, int C_in,
                         int C_out, int L) {
    return cargs(x, xb, L, w, b, out, (long long)C_out * L, L, B, C_in, C_out, L, L, 1, 1, 0);
  }
  // Algorithmic FLOPs / bytes of a launch (each group's input, output,
  // weights, residual, and the read-back of an accumulating combine).
  void conv(const char* t, const ConvLaunch& a) {
    double mac = 0, bytes = 0;
    for (int i = 0; i < a.n_groups; ++i) {
      const ConvGroup& g = a.g[i];
      const double outs = (double)a.B * a.C_out * g.n_out;
      mac += outs * a.C_in * g.K;
      bytes += 4.0 * (outs + (double)a.C_out * a.C_in * g.K);
      if (i == 0 || g.x != a.g[i - 1].x) bytes += 4.0 * (double)a.B * a.C_in * a.L_in;
      if (g.res) bytes += 4.0 * outs;
      if (g.combine != COMB_STORE) bytes += 4.0 * outs;
    }
    const bool b16 = a.g[0].w16 != nullptr;
    const size_t need = b16 ? conv1d_bf16_split_floats(a) : conv1d_mfma_split_floats(a);
    ConvLaunch sa = a;
    if (need > 0) {
      sa.part = buf("splitk", need);
      sa.part_floats = need;
    }
    if (!b16) sa.queue = persist_queue();
    run(t, 2.0 * mac, bytes, [&] {
      if (b16)
        launch_conv1d_bf16(sa, eng->stream);
      else
        launch_conv1d_mfma(sa, eng->stream);
    });
  }
  // the same launch on bf16 weights (row length bf16_ld(C_in)) when w16 is set
  static ConvLaunch with16(ConvLaunch a, const uint16_t* w16) {
    if (w16) {
      a.g[0].w16 = w16;
      a.w16_ld = bf16_ld(a.C_in);
    }
    return a;
  }
};

}  // namespace rvc
