// Device-resident glue around synthesis (rvc_vc_* exports): the steps of
// runtime/pipeline.py that sit either side of SynthesizerTrn.infer --
//   * feature retrieval against a resident index (runtime/retrieval.py:35-83,
//     runtime/pipeline.py:546-566): brute-force L2 k-nearest neighbours as an
//     MFMA GEMM of the queries against the index plus a per-query top-k
//     selection, then the (1/d)^2-weighted blend mixed in at index_rate;
//   * the 2x linear interpolation of the features and the pitch protect mask
//     (runtime/pipeline.py:568-610, runtime/nn.py:734-758);
//   * the RMS envelope mix of the output with the input (runtime/pipeline.py:
//     164-232) and the int16 peak normalisation (:1208-1213).
// A session holds the index (vectors [N][D], their transpose packed as the
// weight operand of the GEMM, and the squared norms) and a workspace reused
// across calls.
#include <cmath>
#include <cstring>

#include "../../include/rvc_hip.h"
#include "session.h"

namespace rvc {

void launch_row_sqnorm(const float* x, float* out, long long rows, int cols, hipStream_t s);
void launch_knn(const float* dot, long long ldd, const float* q2, const float* d2, int F, int N, int k,
                float* part_s, int* part_i, float* scores, long long* inds, hipStream_t s);
size_t knn_part_entries(int F, int N);
void launch_retrieval_blend(const float* scores, const long long* inds, const float* vecs, const float* feats,
                            float* out, int F, int D, int N, int k, float rate, float omr, hipStream_t s);
void launch_interp2_protect(const float* x, const float* x0, const float* pitchf, float protect, float* out, int F,
                            int D, hipStream_t s);
void launch_rms_frames(const float* x, long long n, int hop, float* out, int frames, hipStream_t s);
void launch_rms_mix(const float* data2, long long n2, const float* r1, int L1, const float* r2, int L2, float e1,
                    float e2, float* out, hipStream_t s);
int absmax_parts(long long n);
void launch_to_int16(const float* x, long long n, float* part, short* out, hipStream_t s);

namespace {

constexpr int kK = 8;                           // neighbours per query (runtime/pipeline.py:55)
constexpr size_t kDotBudget = 256ull << 20;     // floats of distance matrix per pass (1 GiB)

struct Vc : SessionBase {
  int N = 0, D = 0, ldN = 0;
  float* vecs = nullptr;  // [N][D]
  float* wT = nullptr;    // [D][ldN]: vecs transposed, columns >= N zero (1x1-conv weight layout)
  float* d2 = nullptr;    // [N]
  std::vector<void*> index_mem;

  ~Vc() override { drop_index(); }

  void drop_index() {
    if (eng && eng->stream) (void)hipStreamSynchronize(eng->stream);
    for (void* p : index_mem) (void)hipFree(p);
    index_mem.clear();
    vecs = wT = d2 = nullptr;
    N = D = ldN = 0;
  }

  float* dalloc(size_t n) {
    void* p = nullptr;
    RVC_HIP(hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(float)));
    index_mem.push_back(p);
    return static_cast<float*>(p);
  }

  void set_index(const float* v, long long n, long long dim) {
    RVC_CHECK(v && n >= 1 && dim >= 1 && n < (1LL << 31) / 2 && dim <= 65536, "set_index: invalid arguments");
    drop_index();
    N = (int)n;
    D = (int)dim;
    ldN = (N + 127) / 128 * 128;
    vecs = dalloc((size_t)N * D);
    RVC_HIP(hipMemcpy(vecs, v, sizeof(float) * (size_t)N * D, hipMemcpyHostToDevice));
    std::vector<float> t((size_t)D * ldN, 0.f);
    for (long long r = 0; r < N; ++r)
      for (long long c = 0; c < D; ++c) t[(size_t)c * ldN + r] = v[r * D + c];
    wT = dalloc(t.size());
    RVC_HIP(hipMemcpy(wT, t.data(), sizeof(float) * t.size(), hipMemcpyHostToDevice));
    d2 = dalloc(N);
    launch_row_sqnorm(vecs, d2, N, D, eng->stream);
    eng->sync();
  }

  // k nearest rows of the index for each query row: scores [F][k] ascending,
  // indices [F][k] (device)
  void search(const float* q, int F, int k, float* scores, long long* inds) {
    RVC_CHECK(N > 0, "search: no index set");
    RVC_CHECK(k >= 1 && k <= kK && k <= N, "search: k must be in [1, min(8, N)]");
    if (F <= 0) return;
    hipStream_t s = eng->stream;
    float* q2 = buf("q2", F);
    launch_row_sqnorm(q, q2, F, D, s);
    float* qT = buf("qT", (size_t)D * F);
    launch_transpose(q, qT, 1, F, D, 1.0f, s);  // [F][D] -> [D][F]
    float* ps = buf("knn_s", knn_part_entries(F, N));
    int* pi = reinterpret_cast<int*>(buf("knn_i", knn_part_entries(F, N)));
    // distance dot products in passes of Fc query columns: dot[n][f] = vecs[n] . q[f]
    const int Fc = (int)std::max<size_t>(1, std::min<size_t>(F, kDotBudget / ldN));
    float* dot = buf("dot", (size_t)ldN * Fc);
    for (int f0 = 0; f0 < F; f0 += Fc) {
      const int fc = std::min(Fc, F - f0);
      ConvLaunch a = c1x1(qT + f0, (long long)D * F, wT, nullptr, dot, 1, D, ldN, fc);
      a.xc = F;  // the pass reads columns f0.. of the full [D][F] transpose
      a.L_in = fc;
      run("vc.knn.gemm", 2.0 * ldN * (double)D * fc, 4.0 * ((double)D * fc + (double)ldN * D + (double)ldN * fc),
          [&] { launch_conv1d_mfma(a, s); });
      run("vc.knn.select", 0.0, 4.0 * (double)ldN * fc, [&] {
        launch_knn(dot, fc, q2 + f0, d2, fc, N, k, ps, pi, scores + (long long)f0 * k, inds + (long long)f0 * k, s);
      });
    }
  }

  // retrieval (when rate != 0 and an index is set), 2x interpolation and the
  // protect mask (pitchf [2F] or null) of feats [F][D] -> out [2F][D]
  void prepare(const float* feats, int F, int Dq, double rate, const float* pitchf, double protect, float* out) {
    if (F <= 0) return;
    hipStream_t s = eng->stream;
    const float* x = feats;
    if (rate != 0.0 && N > 0) {
      RVC_CHECK(Dq == D, "prepare: feature width " + std::to_string(Dq) + " != index width " + std::to_string(D));
      const int k = std::min(kK, N);
      float* sc = buf("sc", (size_t)F * k);
      long long* ix = reinterpret_cast<long long*>(buf("ix", (size_t)F * k * 2));
      search(feats, F, k, sc, ix);
      float* bl = buf("blend", (size_t)F * Dq);
      run("vc.blend", 0.0, 4.0 * 3.0 * F * Dq, [&] {
        launch_retrieval_blend(sc, ix, vecs, feats, bl, F, Dq, N, k, (float)rate, (float)(1.0 - rate), s);
      });
      x = bl;
    }
    run("vc.interp", 0.0, 4.0 * 4.0 * F * Dq, [&] {
      launch_interp2_protect(x, feats, pitchf, (float)protect, out, F, Dq, s);
    });
  }

  void change_rms(const float* d1, long long n1, int sr1, const float* d2in, long long n2, int sr2, double rate,
                  float* out) {
    if (n2 <= 0) return;
    RVC_CHECK(sr1 >= 2 && sr2 >= 2, "change_rms: sample rates must be >= 2");
    hipStream_t s = eng->stream;
    const int h1 = sr1 / 2, h2 = sr2 / 2;
    const long long L1 = 1 + n1 / h1, L2 = 1 + n2 / h2;
    RVC_CHECK(L1 < (1LL << 31) && L2 < (1LL << 31), "change_rms: too many frames");
    float* r1 = buf("rms1", (size_t)L1);
    float* r2 = buf("rms2", (size_t)L2);
    run("vc.rms", 0.0, 4.0 * (double)(n1 + n2), [&] {
      launch_rms_frames(d1, n1, h1, r1, (int)L1, s);
      launch_rms_frames(d2in, n2, h2, r2, (int)L2, s);
      launch_rms_mix(d2in, n2, r1, (int)L1, r2, (int)L2, (float)(1.0 - rate), (float)(rate - 1.0), out, s);
    });
  }

  void to_int16(const float* x, long long n, short* out) {
    if (n <= 0) return;
    float* part = buf("absmax", (size_t)absmax_parts(n));
    run("vc.int16", 0.0, 6.0 * (double)n, [&] { launch_to_int16(x, n, part, out, eng->stream); });
  }
};

std::mutex g_vc_mu;
std::unordered_map<long long, Vc*> g_vcs;
long long g_next_vc = 1;

Vc* vc_from(long long h) {
  std::lock_guard<std::mutex> lk(g_vc_mu);
  auto it = g_vcs.find(h);
  return it == g_vcs.end() ? nullptr : it->second;
}

template <class F>
int32_t vguard(int64_t vh, F&& body) {
  Vc* v = vc_from(vh);
  if (!v) {
    set_last_error("invalid vc handle");
    return -1;
  }
  try {
    std::lock_guard<std::mutex> lk(v->eng->mu);
    body(*v);
    return 0;
  } catch (const std::exception& ex) {
    set_last_error(ex.what());
    return -1;
  }
}

// device copy helper for the host-in / host-out forms
void h2d(void* d, const void* h, size_t bytes, hipStream_t s) {
  if (bytes) RVC_HIP(hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, s));
}
void d2h(void* h, const void* d, size_t bytes, hipStream_t s) {
  if (bytes) RVC_HIP(hipMemcpyAsync(h, d, bytes, hipMemcpyDeviceToHost, s));
}

}  // namespace
}  // namespace rvc

using namespace rvc;

extern "C" {

int64_t rvc_vc_create(int64_t h) {
  Engine* e = engine_from_handle(h);
  if (!e) {
    set_last_error("invalid engine handle");
    return -1;
  }
  Vc* v = new Vc();
  v->eng = e;
  v->ready = true;
  std::lock_guard<std::mutex> lk(g_vc_mu);
  const long long id = g_next_vc++;
  g_vcs[id] = v;
  return id;
}

int32_t rvc_vc_destroy(int64_t vh) {
  Vc* v = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_vc_mu);
    auto it = g_vcs.find(vh);
    if (it == g_vcs.end()) {
      set_last_error("invalid vc handle");
      return -1;
    }
    v = it->second;
    g_vcs.erase(it);
  }
  {
    std::lock_guard<std::mutex> lk(v->eng->mu);
    delete v;
  }
  return 0;
}

int32_t rvc_vc_set_index(int64_t vh, const float* vectors, int64_t n, int64_t dim) {
  return vguard(vh, [&](Vc& v) { v.set_index(vectors, n, dim); });
}

int32_t rvc_vc_index_info(int64_t vh, int64_t* n, int64_t* dim) {
  return vguard(vh, [&](Vc& v) {
    if (n) *n = v.N;
    if (dim) *dim = v.D;
  });
}

int32_t rvc_vc_search(int64_t vh, const float* query, int64_t F, int64_t k, float* scores, int64_t* inds) {
  return vguard(vh, [&](Vc& v) {
    RVC_CHECK(F >= 0 && F < (1LL << 30) && (F == 0 || (query && scores && inds)), "search: invalid arguments");
    if (F == 0) return;
    hipStream_t s = v.eng->stream;
    float* q = v.buf("in_q", (size_t)F * v.D);
    float* sc = v.buf("out_sc", (size_t)F * k);
    long long* ix = reinterpret_cast<long long*>(v.buf("out_ix", (size_t)F * k * 2));
    h2d(q, query, sizeof(float) * (size_t)F * v.D, s);
    v.search(q, (int)F, (int)k, sc, ix);
    v.close_span();
    d2h(scores, sc, sizeof(float) * (size_t)F * k, s);
    d2h(inds, ix, sizeof(long long) * (size_t)F * k, s);
    v.eng->sync();
    v.collect_timing();
  });
}

int32_t rvc_vc_search_dev(int64_t vh, int64_t query, int64_t F, int64_t k, int64_t scores, int64_t inds) {
  return vguard(vh, [&](Vc& v) {
    RVC_CHECK(F >= 0 && F < (1LL << 30), "search: invalid arguments");
    if (F == 0) return;
    Engine& e = *v.eng;
    const float* q = e.fptr(query, F * v.D, "search query");
    float* sc = e.fptr(scores, F * k, "search scores");
    long long* ix = reinterpret_cast<long long*>(e.fptr(inds, F * k * 2, "search indices (int64)"));
    v.search(q, (int)F, (int)k, sc, ix);
    v.close_span();
    e.sync();
    v.collect_timing();
  });
}

int32_t rvc_vc_prepare(int64_t vh, const float* feats, int64_t F, int64_t D, double index_rate, const float* pitchf,
                       double protect, float* out) {
  return vguard(vh, [&](Vc& v) {
    RVC_CHECK(F >= 0 && F < (1LL << 29) && D >= 1 && D <= 65536 && (F == 0 || (feats && out)),
              "prepare: invalid arguments");
    if (F == 0) return;
    hipStream_t s = v.eng->stream;
    float* x = v.buf("in_feats", (size_t)F * D);
    float* pf = pitchf ? v.buf("in_pitchf", (size_t)2 * F) : nullptr;
    float* o = v.buf("out_feats", (size_t)2 * F * D);
    h2d(x, feats, sizeof(float) * (size_t)F * D, s);
    if (pf) h2d(pf, pitchf, sizeof(float) * (size_t)2 * F, s);
    v.prepare(x, (int)F, (int)D, index_rate, pf, protect, o);
    v.close_span();
    d2h(out, o, sizeof(float) * (size_t)2 * F * D, s);
    v.eng->sync();
    v.collect_timing();
  });
}

int32_t rvc_vc_prepare_dev(int64_t vh, int64_t feats, int64_t F, int64_t D, double index_rate, int64_t pitchf,
                           double protect, int64_t out) {
  return vguard(vh, [&](Vc& v) {
    RVC_CHECK(F >= 0 && F < (1LL << 29) && D >= 1 && D <= 65536, "prepare: invalid arguments");
    if (F == 0) return;
    Engine& e = *v.eng;
    const float* x = e.fptr(feats, F * D, "prepare feats");
    const float* pf = pitchf ? e.fptr(pitchf, 2 * F, "prepare pitchf") : nullptr;
    float* o = e.fptr(out, 2 * F * D, "prepare out");
    RVC_CHECK(o != x, "prepare: out must not alias feats");
    v.prepare(x, (int)F, (int)D, index_rate, pf, protect, o);
    v.close_span();
    e.sync();
    v.collect_timing();
  });
}

int32_t rvc_vc_change_rms(int64_t vh, const float* data1, int64_t n1, int64_t sr1, const float* data2, int64_t n2,
                          int64_t sr2, double rate, float* out) {
  return vguard(vh, [&](Vc& v) {
    RVC_CHECK(n1 >= 0 && n2 >= 0 && (n1 == 0 || data1) && (n2 == 0 || (data2 && out)),
              "change_rms: invalid arguments");
    if (n2 == 0) return;
    hipStream_t s = v.eng->stream;
    float* a = v.buf("in_d1", (size_t)std::max<int64_t>(n1, 1));
    float* b = v.buf("in_d2", (size_t)n2);
    float* o = v.buf("out_rms", (size_t)n2);
    h2d(a, data1, sizeof(float) * (size_t)n1, s);
    h2d(b, data2, sizeof(float) * (size_t)n2, s);
    v.change_rms(a, n1, (int)sr1, b, n2, (int)sr2, rate, o);
    v.close_span();
    d2h(out, o, sizeof(float) * (size_t)n2, s);
    v.eng->sync();
    v.collect_timing();
  });
}

int32_t rvc_vc_change_rms_dev(int64_t vh, int64_t data1, int64_t n1, int64_t sr1, int64_t data2, int64_t n2,
                              int64_t sr2, double rate, int64_t out) {
  return vguard(vh, [&](Vc& v) {
    RVC_CHECK(n1 >= 0 && n2 >= 0, "change_rms: invalid arguments");
    if (n2 == 0) return;
    Engine& e = *v.eng;
    const float* a = n1 ? e.fptr(data1, n1, "change_rms data1") : nullptr;
    const float* b = e.fptr(data2, n2, "change_rms data2");
    float* o = e.fptr(out, n2, "change_rms out");
    v.change_rms(a, n1, (int)sr1, b, n2, (int)sr2, rate, o);
    v.close_span();
    e.sync();
    v.collect_timing();
  });
}

int32_t rvc_vc_to_int16(int64_t vh, const float* x, int64_t n, int16_t* out) {
  return vguard(vh, [&](Vc& v) {
    RVC_CHECK(n >= 0 && (n == 0 || (x && out)), "to_int16: invalid arguments");
    if (n == 0) return;
    hipStream_t s = v.eng->stream;
    float* a = v.buf("in_x", (size_t)n);
    short* o = reinterpret_cast<short*>(v.buf("out_i16", (size_t)(n + 1) / 2));
    h2d(a, x, sizeof(float) * (size_t)n, s);
    v.to_int16(a, n, o);
    v.close_span();
    d2h(out, o, sizeof(short) * (size_t)n, s);
    v.eng->sync();
    v.collect_timing();
  });
}

int32_t rvc_vc_to_int16_dev(int64_t vh, int64_t x, int64_t n, int64_t out) {
  return vguard(vh, [&](Vc& v) {
    RVC_CHECK(n >= 0, "to_int16: invalid arguments");
    if (n == 0) return;
    Engine& e = *v.eng;
    const float* a = e.fptr(x, n, "to_int16 x");
    DevBuf& ob = e.get(out);
    RVC_CHECK(ob.bytes >= (size_t)n * 2, "to_int16 out: buffer too small (int16 [n])");
    v.to_int16(a, n, static_cast<short*>(ob.ptr));
    v.close_span();
    e.sync();
    v.collect_timing();
  });
}

int32_t rvc_vc_set_timing(int64_t vh, const char* tag) {
  return vguard(vh, [&](Vc& v) { v.set_timing(tag); });
}

int32_t rvc_vc_get_timing(int64_t vh, double* total_ms, int64_t* launches, double* flops, double* bytes) {
  return vguard(vh, [&](Vc& v) {
    if (total_ms) *total_ms = v.t_ms;
    if (launches) *launches = v.t_n;
    if (flops) *flops = v.t_flops;
    if (bytes) *bytes = v.t_bytes;
  });
}

}  // extern "C"
