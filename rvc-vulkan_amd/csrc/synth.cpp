// Device-resident RVC v2 synthesis session (rvc_synth_* exports).
//
// Holds the packed weights of one SynthesizerTrnMs*NSFsid and runs
//   enc_p   runtime/models/vits.py:499-538, 962-1059   (TextEncoder)
//   flow    runtime/models/vits.py:1086-1145, 1255-1268 (reverse coupling)
//   dec     runtime/models/vits.py:1468-1501, 2133-2231 (GeneratorNSF)
// composed as in SynthesizerTrn.infer_controlled (:2551-2595), every op a
// HIP kernel on the engine stream, intermediates resident in HBM.
//
// Fusions relative to the reference's op sequence:
//   * conv_pre + bias + cond(g) in one conv epilogue (bias2 term);
//   * noise conv written first, each ConvTranspose phase accumulates on top
//     (x = ups(lrelu(x)) + noise_conv(har)), the leaky-ReLU applied while the
//     input tile is staged;
//   * each ResBlock conv applies leaky-ReLU on load and on store, the second
//     conv adds the residual; the three ResBlocks of a stage share every
//     conv launch (one grid per dilation group) and are averaged as
//     ((o_3 + o_7) + o_11) / 3 (the numpy order of :2225-2227);
//   * conv_o / FFN conv_2 add the encoder residual in their epilogue; FFN
//     conv_1 applies ReLU on store;
//   * windowed relative-position attention is one kernel (attention.hip).
//
// Precision modes (rvc_synth_set_precision, before finalize): 0 = fp32
// everywhere; 1 = the GeneratorNSF upsample ConvTranspose1d and the enc_p
// matmuls (pitch/phone embedding linear, q/k/v, conv_o, FFN, proj) on bf16
// MFMA with fp32 accumulate; 2 = mode 1 plus the
// decoder ResBlock convs on bf16.  Everything else stays fp32.
#include <algorithm>
#include <functional>
#include <cmath>
#include <cstring>

#include "../../include/rvc_hip.h"
#include "session.h"

namespace rvc {

struct Synth : SessionBase {

  // ---- geometry (VitsConfig, runtime/models/vits.py:166-268) ----
  int phone_dim = 0, H = 0, F = 0, n_layers = 0, heads = 0, kc = 0, gin = 0, n_spk = 0;
  int U = 0, n_ups = 0, upp = 0, sr = 0, half = 0, n_flows = 0, pitch_rows = 0;
  static constexpr int kWnLayers = 3, kWnKernel = 5, kWindow = 10;
  std::vector<int> rates, kernels, chans, noise_k, noise_s;

  // ---- device weights ----
  float *emb_phone_w = nullptr, *emb_phone_b = nullptr, *emb_pitch = nullptr, *emb_g = nullptr;
  struct EncL {
    float *wqkv, *bqkv, *wo, *bo, *ek, *ev, *g1, *b1, *w1, *bf1, *w2, *bf2, *g2, *b2;
    float* wo_lanes;  // conv_o in pack_mfma_lanes order (attn_out_ln_kernel), or null
    uint16_t *wqkv16, *wo16, *w116, *w216;  // bf16 copies (precision >= 1), else null
  };
  std::vector<EncL> enc;
  float *proj_w = nullptr, *proj_b = nullptr;
  uint16_t *emb_phone16 = nullptr, *proj16 = nullptr;
  int precision = 0;
  // A flow entered with its channels reversed relative to the reference's
  // (see flow()) reads the pre conv's half with the weight's input channels
  // reversed, and subtracts the post conv's rows in reverse order.
  struct FlowL {
    bool rev;
    float *pre_w, *pre_b, *post_w, *post_b;
    float *in_w[kWnLayers], *in_b[kWnLayers], *rs_w[kWnLayers], *rs_b[kWnLayers];
    int rs_out[kWnLayers];
    // the flow tail's weights in pack_mfma_lanes order (null when H does not
    // take the flow tail): the last res/skip conv, post, pre
    float *rs_lanes, *post_lanes, *pre_lanes;
  };
  std::vector<FlowL> flows;
  // every flow's cond_layer stacked, [n_flows * 2H * kWnLayers][gin]
  float *flow_cond_w = nullptr, *flow_cond_b = nullptr;
  float *dpre_w = nullptr, *dpre_b = nullptr, *dcond_w = nullptr, *dcond_b = nullptr, *dpost_w = nullptr;
  float w_lin = 0.f, b_lin = 0.f;
  struct StageW {
    std::vector<float*> phases;
    float* up_b;
    float *nw, *nb;
    float* rw[3][2][3];
    float* rb[3][2][3];
    std::vector<uint16_t*> phases16;  // precision >= 1
    uint16_t* rw16[3][2][3];          // precision 2, else null
    // fp32 output-stationary ConvTranspose (convt_os_supported shapes): all
    // taps packed [K][C_in][packed_ld(C)]; null when the polyphase grids run
    float* up_all = nullptr;
    // bf16 output-stationary ConvTranspose (precision >= 1): all taps packed
    // [K][C_out][bf16_ld(C_in)] in bf16; null when the polyphase grids run
    uint16_t* up_all16 = nullptr;
    bool noise_fused = false;  // the stage's noise conv is computed by that kernel
  };
  std::vector<StageW> stages;

  // ---- side stream ----
  // The NSF source, the noise convs and the decoder's cond projection depend
  // only on f0, the noise and g, so they run on a second (default-priority)
  // stream while enc_p and flow run on the engine stream; conv_pre waits on
  // `joined`. Each upsample stage keeps its noise conv output in a buffer of
  // its own (dN<i>), into which the ConvTranspose then accumulates.
  hipStream_t side = nullptr;
  hipEvent_t forked = nullptr, joined = nullptr;
  float* dec_cv = nullptr;
  float* dec_har = nullptr;  // the harmonic source of the current call (side stream)
  std::vector<float*> dec_noise;

  // ---- deferred calls (rvc_synth_submit / _collect / _abort) ----
  // Each outstanding call owns a pinned host staging buffer and an event
  // recorded after its waveform's device-to-host copy; the calls share the
  // workspace, which the one engine stream keeps in order.
  struct Pending {
    long long id = 0;  // 0: free
    float* host = nullptr;
    size_t cap = 0;    // floats
    hipEvent_t done = nullptr;
    long long n = 0;   // floats of this call's waveform
  };
  std::vector<Pending> pend;
  long long next_ticket = 1;
  static constexpr int kMaxPending = 8;
  void pending_room() const {
    int busy = 0;
    for (const Pending& p : pend) busy += p.id != 0;
    RVC_CHECK(busy < kMaxPending, "submit: too many outstanding calls (collect or abort some first)");
  }
  // reserve a free slot for a call whose work is already queued
  Pending& pending_slot(long long n) {
    Pending* slot = nullptr;
    for (Pending& p : pend)
      if (p.id == 0) {
        slot = &p;
        break;
      }
    if (!slot) {
      RVC_CHECK((int)pend.size() < kMaxPending, "submit: too many outstanding calls (collect or abort some first)");
      pend.emplace_back();
      slot = &pend.back();
      RVC_HIP(hipEventCreateWithFlags(&slot->done, hipEventDisableTiming));
    }
    if (slot->cap < (size_t)n) {
      if (slot->host) RVC_HIP(hipHostFree(slot->host));
      slot->host = nullptr;
      slot->cap = 0;
      RVC_HIP(hipHostMalloc((void**)&slot->host, sizeof(float) * std::max<long long>(n, 1), hipHostMallocDefault));
      slot->cap = (size_t)n;
    }
    slot->id = next_ticket++;
    slot->n = n;
    return *slot;
  }
  Pending& pending_find(long long id) {
    for (Pending& p : pend)
      if (id > 0 && p.id == id) return p;
    RVC_CHECK(false, "collect: unknown or already collected ticket");
    return pend.front();  // not reached
  }

  ~Synth() override {
    for (Pending& p : pend) {
      if (p.done) {
        (void)hipEventSynchronize(p.done);
        (void)hipEventDestroy(p.done);
      }
      if (p.host) (void)hipHostFree(p.host);
    }
    if (side) (void)hipStreamSynchronize(side);
    if (forked) (void)hipEventDestroy(forked);
    if (joined) (void)hipEventDestroy(joined);
    if (side) (void)hipStreamDestroy(side);
    if (errh) (void)hipHostFree(errh);
  }

  // ---- id validation on the device path ----
  // The pitch / speaker gathers of a call whose ids live in device memory set
  // bits of errw for ids outside [-rows, rows); the word is cleared at the
  // start of the call and copied to pinned host memory before its final
  // synchronisation, so checking it costs no extra round trip.
  unsigned* errw = nullptr;
  unsigned* errh = nullptr;
  void begin_ids() {
    if (!errw) {
      void* p = nullptr;
      RVC_HIP(hipMalloc(&p, 256));
      owned.push_back(p);
      errw = static_cast<unsigned*>(p);
      RVC_HIP(hipHostMalloc((void**)&errh, sizeof(unsigned), hipHostMallocDefault));
    }
    *errh = 0;
    launch_fill(reinterpret_cast<float*>(errw), 1, 0.f, eng->stream);  // +0.0f is the bit pattern 0
  }
  void fetch_ids() { RVC_HIP(hipMemcpyAsync(errh, errw, sizeof(unsigned), hipMemcpyDeviceToHost, eng->stream)); }
  // after the call's synchronisation
  void check_ids() const {
    RVC_CHECK(!(*errh & 1u), "infer: pitch id out of range");
    RVC_CHECK(!(*errh & 2u), "infer: sid out of range");
  }

  // ---- workspace ----
  bool keep_stages = false;
  std::string z_name = "z_p";  // workspace buffer holding the last flow output

  // -------------------------------------------------------------- weights
  std::vector<float> deweight(const std::string& base) const {
    // W = v * (g / max(||v||, 1e-12)), norm over all dims but 0
    // (runtime/models/vits.py:416-442)
    const HostT& v = W(base + ".weight_v");
    const HostT& g = W(base + ".weight_g");
    const long long d0 = v.shape[0];
    const long long per = (long long)v.data.size() / d0;
    RVC_CHECK((long long)g.data.size() == d0, base + ".weight_g: expected one scale per output channel");
    std::vector<float> out(v.data.size());
    for (long long o = 0; o < d0; ++o) {
      double s = 0;
      for (long long j = 0; j < per; ++j) s += (double)v.data[o * per + j] * v.data[o * per + j];
      float norm = (float)std::sqrt(s);
      norm = std::max(norm, 1e-12f);
      const float scale = g.data[o] / norm;
      for (long long j = 0; j < per; ++j) out[o * per + j] = v.data[o * per + j] * scale;
    }
    return out;
  }

  std::vector<float> conv_host(const std::string& key, long long C_out, long long C_in, long long K, bool wn) const {
    if (wn) {
      const HostT& v = W(key + ".weight_v");
      check_shape(key + ".weight_v", v.shape, {C_out, C_in, K});
      return deweight(key);
    }
    const HostT& t = W(key + ".weight");
    check_shape(key + ".weight", t.shape, {C_out, C_in, K});
    return t.data;
  }
  float* upload_conv(const std::string& key, long long C_out, long long C_in, long long K, bool wn) {
    return upload(pack(conv_host(key, C_out, C_in, K, wn), C_out, C_in, K));
  }
  // bf16 copy of a conv weight when `on`, else null
  uint16_t* upload_conv16(bool on, const std::string& key, long long C_out, long long C_in, long long K, bool wn) {
    return on ? upload16(pack_bf16(conv_host(key, C_out, C_in, K, wn), C_out, C_in, K)) : nullptr;
  }

  void finalize(int sr_, const std::vector<int>& rates_, const std::vector<int>& kernels_) {
    RVC_CHECK(!ready, "synth session already finalized");
    sr = sr_;
    rates = rates_;
    kernels = kernels_;
    n_ups = (int)rates.size();
    RVC_CHECK(n_ups >= 1 && kernels.size() == rates.size(), "finalize: need matching upsample rates/kernels");
    const HostT& ep = W("enc_p.emb_phone.weight");
    RVC_CHECK(ep.shape.size() == 2, "enc_p.emb_phone.weight must be 2-D");
    H = (int)ep.shape[0];
    phone_dim = (int)ep.shape[1];
    F = (int)W("enc_p.encoder.ffn_layers.0.conv_1.weight").shape[0];
    while (has("enc_p.encoder.attn_layers." + std::to_string(n_layers) + ".conv_q.weight")) ++n_layers;
    const HostT& erk = W("enc_p.encoder.attn_layers.0.emb_rel_k");
    RVC_CHECK(erk.shape.size() == 3 && erk.shape[1] == 2 * kWindow + 1, "emb_rel_k must be [1, 21, k_channels]");
    kc = (int)erk.shape[2];
    heads = H / kc;
    RVC_CHECK(heads * kc == H, "hidden must be a multiple of k_channels");
    const HostT& eg = W("emb_g.weight");
    n_spk = (int)eg.shape[0];
    gin = (int)eg.shape[1];
    U = (int)W("dec.conv_pre.weight").shape[0];
    pitch_rows = (int)W("enc_p.emb_pitch.weight").shape[0];
    half = H / 2;
    upp = 1;
    for (int r : rates) {
      RVC_CHECK(r >= 1, "upsample rates must be >= 1");
      upp *= r;
    }
    while (has("flow.flows." + std::to_string(2 * n_flows) + ".pre.weight")) ++n_flows;

    // ---- enc_p ----
    check_shape("enc_p.emb_phone.weight", ep.shape, {H, phone_dim});
    const bool b16 = precision >= 1;
    emb_phone_w = upload(pack(ep.data, H, phone_dim, 1));
    emb_phone16 = b16 ? upload16(pack_bf16(ep.data, H, phone_dim, 1)) : nullptr;
    emb_phone_b = upload_vec("enc_p.emb_phone.bias", H);
    check_shape("enc_p.emb_pitch.weight", W("enc_p.emb_pitch.weight").shape, {pitch_rows, H});
    emb_pitch = upload_key("enc_p.emb_pitch.weight");
    emb_g = upload_key("emb_g.weight");
    for (int i = 0; i < n_layers; ++i) {
      const std::string a = "enc_p.encoder.attn_layers." + std::to_string(i);
      EncL L{};
      std::vector<float> qkv, bqkv;
      for (const char* nm : {"conv_q", "conv_k", "conv_v"}) {
        const HostT& t = W(a + "." + nm + ".weight");
        check_shape(a + "." + nm + ".weight", t.shape, {H, H, 1});
        qkv.insert(qkv.end(), t.data.begin(), t.data.end());
        const HostT& b = W(a + "." + nm + ".bias");
        RVC_CHECK((int)b.data.size() == H, a + "." + nm + ".bias size");
        bqkv.insert(bqkv.end(), b.data.begin(), b.data.end());
      }
      L.wqkv = upload(pack(qkv, 3 * H, H, 1));
      L.wqkv16 = b16 ? upload16(pack_bf16(qkv, 3 * H, H, 1)) : nullptr;
      L.wo16 = upload_conv16(b16, a + ".conv_o", H, H, 1, false);
      L.bqkv = upload(bqkv);
      L.wo = upload_conv(a + ".conv_o", H, H, 1, false);
      L.wo_lanes = H % 16 == 0 ? upload(pack_mfma_lanes(conv_host(a + ".conv_o", H, H, 1, false), H, H)) : nullptr;
      L.bo = upload_vec(a + ".conv_o.bias", H);
      check_shape(a + ".emb_rel_k", W(a + ".emb_rel_k").shape, {1, 2 * kWindow + 1, kc});
      check_shape(a + ".emb_rel_v", W(a + ".emb_rel_v").shape, {1, 2 * kWindow + 1, kc});
      L.ek = upload_key(a + ".emb_rel_k");
      L.ev = upload_key(a + ".emb_rel_v");
      const std::string n1 = "enc_p.encoder.norm_layers_1." + std::to_string(i);
      const std::string n2 = "enc_p.encoder.norm_layers_2." + std::to_string(i);
      L.g1 = upload_vec(n1 + ".gamma", H);
      L.b1 = upload_vec(n1 + ".beta", H);
      L.g2 = upload_vec(n2 + ".gamma", H);
      L.b2 = upload_vec(n2 + ".beta", H);
      const std::string f = "enc_p.encoder.ffn_layers." + std::to_string(i);
      L.w1 = upload_conv(f + ".conv_1", F, H, 3, false);
      L.w116 = upload_conv16(b16, f + ".conv_1", F, H, 3, false);
      L.w216 = upload_conv16(b16, f + ".conv_2", H, F, 3, false);
      L.bf1 = upload_vec(f + ".conv_1.bias", F);
      L.w2 = upload_conv(f + ".conv_2", H, F, 3, false);
      L.bf2 = upload_vec(f + ".conv_2.bias", H);
      enc.push_back(L);
    }
    proj_w = upload_conv("enc_p.proj", 2 * H, H, 1, false);
    proj16 = upload_conv16(b16, "enc_p.proj", 2 * H, H, 1, false);
    proj_b = upload_vec("enc_p.proj.bias", 2 * H);

    // ---- flow ----
    const long long GW = 2LL * H * kWnLayers;  // cond rows per flow
    std::vector<float> cond_w, cond_b;
    for (int fi = 0; fi < n_flows; ++fi) {
      const std::string b = "flow.flows." + std::to_string(2 * fi);
      FlowL L{};
      // flow() runs the flows from the last to the first, the channel order
      // reversed (relative to the reference's) on the 1st, 3rd, ... of them
      L.rev = ((n_flows - fi) & 1) != 0;
      std::vector<float> pw = conv_host(b + ".pre", H, half, 1, false);
      std::vector<float> qw = conv_host(b + ".post", half, H, 1, false);
      std::vector<float> qb = W(b + ".post.bias").data;
      RVC_CHECK((long long)qb.size() == half, "weight " + b + ".post.bias must hold " + std::to_string(half) + " values");
      if (L.rev) {
        for (long long o = 0; o < H; ++o) std::reverse(pw.begin() + o * half, pw.begin() + (o + 1) * half);
        std::vector<float> rq(qw.size());
        for (long long o = 0; o < half; ++o)
          std::copy(qw.begin() + (half - 1 - o) * H, qw.begin() + (half - o) * H, rq.begin() + o * H);
        qw.swap(rq);
        std::reverse(qb.begin(), qb.end());
      }
      L.pre_w = upload(pack(pw, H, half, 1));
      L.pre_b = upload_vec(b + ".pre.bias", H);
      L.post_w = upload(pack(qw, half, H, 1));
      if (flow_tail_supported(H, half)) {
        L.pre_lanes = upload(pack_mfma_lanes(pw, H, half));
        L.post_lanes = upload(pack_mfma_lanes(qw, half, H));
      }
      L.post_b = upload(qb);
      const HostT& cv = W(b + ".enc.cond_layer.weight_v");
      check_shape(b + ".enc.cond_layer.weight_v", cv.shape, {GW, gin, 1});
      const std::vector<float> cw = deweight(b + ".enc.cond_layer");
      cond_w.insert(cond_w.end(), cw.begin(), cw.end());
      const HostT& cb = W(b + ".enc.cond_layer.bias");
      RVC_CHECK((long long)cb.data.size() == GW, "weight " + b + ".enc.cond_layer.bias has the wrong size");
      cond_b.insert(cond_b.end(), cb.data.begin(), cb.data.end());
      for (int i = 0; i < kWnLayers; ++i) {
        const std::string il = b + ".enc.in_layers." + std::to_string(i);
        L.in_w[i] = upload_conv(il, 2 * H, H, kWnKernel, true);
        L.in_b[i] = upload_vec(il + ".bias", 2 * H);
        const std::string rl = b + ".enc.res_skip_layers." + std::to_string(i);
        L.rs_out[i] = i < kWnLayers - 1 ? 2 * H : H;
        L.rs_w[i] = upload_conv(rl, L.rs_out[i], H, 1, true);
        L.rs_b[i] = upload_vec(rl + ".bias", L.rs_out[i]);
        if (i == kWnLayers - 1 && flow_tail_supported(H, half))
          L.rs_lanes = upload(pack_mfma_lanes(conv_host(rl, L.rs_out[i], H, 1, true), H, H));
      }
      flows.push_back(L);
    }
    flow_cond_w = upload(cond_w);
    flow_cond_b = upload(cond_b);

    // ---- dec ----
    dpre_w = upload_conv("dec.conv_pre", U, H, 7, false);
    dpre_b = upload_vec("dec.conv_pre.bias", U);
    check_shape("dec.cond.weight", W("dec.cond.weight").shape, {U, gin, 1});
    dcond_w = upload_key("dec.cond.weight");
    dcond_b = upload_vec("dec.cond.bias", U);
    RVC_CHECK(W("dec.m_source.l_linear.weight").data.size() == 1 && W("dec.m_source.l_linear.bias").data.size() == 1,
              "dec.m_source.l_linear must be 1x1");
    w_lin = W("dec.m_source.l_linear.weight").data[0];
    b_lin = W("dec.m_source.l_linear.bias").data[0];
    int c_in = U;
    for (int i = 0; i < n_ups; ++i) {
      const std::string up = "dec.ups." + std::to_string(i);
      const HostT& v = W(up + ".weight_v");
      RVC_CHECK(v.shape.size() == 3 && v.shape[0] == c_in && v.shape[2] == kernels[i],
                up + ".weight_v must be [C_in, C_out, K]");
      const int c = (int)v.shape[1];
      RVC_CHECK(c == U >> (i + 1), up + ": stage channels must be upsample_initial / 2^(i+1)");
      chans.push_back(c);
      StageW S{};
      const std::vector<float> wt = deweight(up);
      const int K = kernels[i], st = rates[i];
      RVC_CHECK(st <= kMaxConvGroups && (K + st - 1) / st <= kConvTapsMax, up + ": stride / taps unsupported");
      const int ld = packed_ld(c);
      for (int r = 0; r < st; ++r) {
        const int J = convt_phase_taps(K, st, r);
        std::vector<float> ph((size_t)J * c_in * ld, 0.f);
        for (int jp = 0; jp < J; ++jp) {
          const int k = r + (J - 1 - jp) * st;
          for (int ci = 0; ci < c_in; ++ci)
            for (int co = 0; co < c; ++co)
              ph[((size_t)jp * c_in + ci) * ld + co] = wt[((size_t)ci * c + co) * K + k];
        }
        S.phases.push_back(upload(ph));
        if (b16 && !(convt_os_supported(K, st) && c_in % 32 == 0 && c % 32 == 0)) {
          const int ld16 = bf16_ld(c_in);
          std::vector<uint16_t> p16((size_t)J * c * ld16, 0);
          for (int jp = 0; jp < J; ++jp) {
            const int k = r + (J - 1 - jp) * st;
            for (int co = 0; co < c; ++co)
              for (int ci = 0; ci < c_in; ++ci)
                p16[((size_t)jp * c + co) * ld16 + ci] = f32_to_bf16(wt[((size_t)ci * c + co) * K + k]);
          }
          S.phases16.push_back(upload16(p16));
        }
      }
      S.up_b = upload_vec(up + ".bias", c);
      const std::string nc = "dec.noise_convs." + std::to_string(i);
      const HostT& nw = W(nc + ".weight");
      RVC_CHECK(nw.shape.size() == 3 && nw.shape[0] == c && nw.shape[1] == 1, nc + ".weight must be [C, 1, k]");
      const int kn = (int)nw.shape[2];
      noise_k.push_back(kn);
      noise_s.push_back(i < n_ups - 1 ? kn / 2 : 1);
      if (!b16 && convt_os_supported(K, st) && c_in % 8 == 0 && c % 32 == 0) {
        std::vector<float> all((size_t)K * c_in * ld, 0.f);  // [k][ci][co] = wt[ci][co][k]
        for (int k = 0; k < K; ++k)
          for (int ci = 0; ci < c_in; ++ci)
            for (int co = 0; co < c; ++co) all[((size_t)k * c_in + ci) * ld + co] = wt[((size_t)ci * c + co) * K + k];
        S.up_all = upload(all);
        S.noise_fused = kn <= kNoiseTapsMax;
      }
      if (b16 && convt_os_supported(K, st) && c_in % 32 == 0 && c % 32 == 0) {
        const int ld16 = bf16_ld(c_in);
        std::vector<uint16_t> all16((size_t)K * c * ld16, 0);  // [k][co][ci] = bf16(wt[ci][co][k])
        for (int k = 0; k < K; ++k)
          for (int co = 0; co < c; ++co)
            for (int ci = 0; ci < c_in; ++ci)
              all16[((size_t)k * c + co) * ld16 + ci] = f32_to_bf16(wt[((size_t)ci * c + co) * K + k]);
        S.up_all16 = upload16(all16);
        S.noise_fused = kn <= kNoiseTapsMax;
      }
      S.nw = upload_key(nc + ".weight");
      S.nb = upload_vec(nc + ".bias", c);
      static const int ks[3] = {3, 7, 11};
      for (int j = 0; j < 3; ++j)
        for (int l = 0; l < 2; ++l)
          for (int g = 0; g < 3; ++g) {
            const std::string rb = "dec.resblocks." + std::to_string(3 * i + j) + (l == 0 ? ".convs1." : ".convs2.") +
                                   std::to_string(g);
            S.rw[j][l][g] = upload_conv(rb, c, c, ks[j], true);
            S.rw16[j][l][g] = upload_conv16(precision >= 2, rb, c, c, ks[j], true);
            S.rb[j][l][g] = upload_vec(rb + ".bias", c);
          }
      stages.push_back(S);
      c_in = c;
    }
    check_shape("dec.conv_post.weight", W("dec.conv_post.weight").shape, {1, c_in, 7});
    dpost_w = upload_key("dec.conv_post.weight");
    host.clear();
    ready = true;
  }

  // stage lengths and the decoder ping-pong capacity for P frames
  size_t dec_cap(int P) const {
    size_t cap = (size_t)U * P;
    long long L = P;
    for (int i = 0; i < n_ups; ++i) {
      L *= rates[i];
      cap = std::max(cap, (size_t)(chans[i] * L));
    }
    return cap;
  }

  // -------------------------------------------------------------- enc_p + flow
  // g [B][gin] = emb_g(sid)
  void speaker(const long long* sid, int B, float* g) {
    run("enc.glue", 0.0, 8.0 * B + 8.0 * B * gin,
        [&] { launch_gather_rows_i64(sid, emb_g, g, B, n_spk, gin, errw, eng->stream); });
  }

  // Whether enc_p runs the fused five-launch layers: fp32, at least one
  // layer, H within the staged-LayerNorm 1x1 kernel and the fused attention
  // output kernel, P within the whole-reduction kernels' column limit.
  bool fused_layers(int P) const {
    return precision == 0 && n_layers > 0 && H <= 256 && H % 8 == 0 && P <= 8192 &&
           attn_out_ln_supported(heads, kc, relpos_attention_splits(heads, kc, P, kWindow, true));
  }
  // a 1x1 conv whose input is the un-normalised sum before layer L's second
  // LayerNorm: normalise while staging, and store the normalised tensor
  static void stage_ln(ConvLaunch& c, const EncL& L, float* out, long long HP, int P) {
    c.ln_g = L.g2;
    c.ln_b = L.b2;
    c.ln_out = out;
    c.ln_ob = HP;
    c.ln_oc = P;
    c.ln_eps = 1e-5f;
  }

  // enc_p: embedding, the attention / FFN layers and proj, then
  // z_p = m + exp(logs) * nz * 0.66666 -> [B][H][P] (batch stride H*P).
  // before_zp (optional) runs on the host once every enc_p kernel but z_p is
  // queued: the host-input path uploads nz (and the decoder's f0 / noise)
  // there, so those copies overlap the encoder on the GPU.
  float* encode(const float* phone, const long long* pitch, const float* nz, int B, int P,
                const std::function<void()>& before_zp = {}) {
    hipStream_t s = eng->stream;
    const long long HP = (long long)H * P;
    float* phT = buf("phT", (size_t)B * phone_dim * P);
    run("enc.glue", 0.0, 8.0 * B * phone_dim * P, [&] { launch_transpose(phone, phT, B, P, phone_dim, 1.0f, s); });
    float* E = buf("encE", (size_t)B * HP);
    conv("enc.embed", with16(c1x1(phT, (long long)phone_dim * P, emb_phone_w, emb_phone_b, E, B, phone_dim, H, P),
                             emb_phone16));
    float* xin = buf("enc_in", (size_t)B * HP);
    run("enc.glue", 0.0, 4.0 * B * (3.0 * HP + 2.0 * P), [&] {
      launch_embed_combine(E, pitch, emb_pitch, pitch_rows, xin, B, H, P, (float)std::sqrt((double)H), 0.1f, errw, s);
    });
    float* xo = buf("enc_out", (size_t)B * HP);
    float* qkv = buf("qkv", (size_t)B * 3 * HP);
    float* att = buf("att", (size_t)B * HP);
    float* o = buf("enco", (size_t)B * HP);
    float* f = buf("ffn", (size_t)B * F * P);
    const size_t apart_n = std::max<size_t>(1, relpos_attention_scratch_floats(B, heads, kc, P, kWindow, true));
    float* apart = buf("attn_part", apart_n);
    if (fused_layers(P)) {
      // Five launches per layer: q/k/v (with the previous layer's second
      // LayerNorm applied while its input is staged; its C_out tile 0 also
      // stores the normalised tensor, the layer's residual), the attention,
      // merge + conv_o + residual + LayerNorm in one kernel, the two FFN
      // convs (the second adds the residual and leaves its sum
      // un-normalised for the next consumer).  proj applies the last
      // LayerNorm the same way and stores enc_out.
      float* x1 = buf("enc_x1", (size_t)B * HP);
      const int KS = relpos_attention_splits(heads, kc, P, kWindow, true);
      for (int i = 0; i < n_layers; ++i) {
        const EncL& L = enc[i];
        ConvLaunch cq = c1x1(i == 0 ? xin : o, HP, L.wqkv, L.bqkv, qkv, B, H, 3 * H, P);
        if (i > 0) stage_ln(cq, enc[i - 1], xo, HP, P);
        conv("enc.qkv", cq);
        run("enc.attn", 4.0 * B * heads * (double)P * P * kc, 4.0 * B * 4 * HP, [&] {
          const int ks = launch_relpos_attention_partials(qkv, L.ek, L.ev, att, apart, apart_n, B, heads, kc, P,
                                                          kWindow, s);
          RVC_CHECK(ks == KS, "encode: attention key split changed");
        });
        AttnOutArgs ao{};
        ao.part = apart;
        ao.att = att;
        ao.w = L.wo_lanes;
        ao.bias = L.bo;
        ao.res = i == 0 ? xin : xo;
        ao.g = L.g1;
        ao.beta = L.b1;
        ao.out = x1;
        ao.H = heads;
        ao.D = kc;
        ao.P = P;
        ao.KS = KS;
        ao.eps = 1e-5f;
        const double in_bytes = KS > 1 ? 4.0 * B * heads * KS * (kc + 2.0) * P : 4.0 * B * HP;
        run("enc.o", 2.0 * B * H * (double)H * P, in_bytes + 4.0 * (3.0 * B * HP + (double)H * H),
            [&] { launch_attn_out_ln(ao, B, s); });
        ConvLaunch c1 = cargs_same(x1, HP, P, L.w1, L.bf1, f, (long long)F * P, P, B, H, F, P, 3, 1, 1);
        c1.out_act = ACT_RELU;
        conv("enc.ffn", c1);
        ConvLaunch c2 = cargs_same(f, (long long)F * P, P, L.w2, L.bf2, o, HP, P, B, F, H, P, 3, 1, 1);
        c2.g[0].res = x1; c2.rb = HP; c2.rc = P;
        conv("enc.ffn", c2);
      }
      float* st = buf("stats", (size_t)B * 2 * HP);
      ConvLaunch cp = c1x1(o, HP, proj_w, proj_b, st, B, H, 2 * H, P);
      stage_ln(cp, enc[n_layers - 1], xo, HP, P);
      conv("enc.proj", cp);
      float* zp = buf("z_p", (size_t)B * HP);
      if (before_zp) before_zp();
    run("enc.glue", 3.0 * B * HP, 16.0 * B * HP, [&] { launch_zp(st, nz, zp, B, H, P, 0.66666f, s); });
      return zp;
    }
    const float* x = xin;
    for (int i = 0; i < n_layers; ++i) {
      const EncL& L = enc[i];
      conv("enc.qkv", with16(c1x1(x, HP, L.wqkv, L.bqkv, qkv, B, H, 3 * H, P), L.wqkv16));
      run("enc.attn", 4.0 * B * heads * (double)P * P * kc, 4.0 * B * 4 * HP,
          [&] { launch_relpos_attention(qkv, L.ek, L.ev, att, apart, apart_n, B, heads, kc, P, kWindow, s); });
      ConvLaunch co = with16(c1x1(att, HP, L.wo, L.bo, o, B, H, H, P), L.wo16);
      co.g[0].res = x; co.rb = HP; co.rc = P;
      conv("enc.o", co);
      run("enc.ln", 8.0 * B * HP, 8.0 * B * HP, [&] { launch_layernorm_cols(o, L.g1, L.b1, xo, B, H, P, 1e-5f, s); });
      ConvLaunch c1 = with16(cargs_same(xo, HP, P, L.w1, L.bf1, f, (long long)F * P, P, B, H, F, P, 3, 1, 1), L.w116);
      c1.out_act = ACT_RELU;
      conv("enc.ffn", c1);
      ConvLaunch c2 = with16(cargs_same(f, (long long)F * P, P, L.w2, L.bf2, o, HP, P, B, F, H, P, 3, 1, 1), L.w216);
      c2.g[0].res = xo; c2.rb = HP; c2.rc = P;
      conv("enc.ffn", c2);
      run("enc.ln", 8.0 * B * HP, 8.0 * B * HP, [&] { launch_layernorm_cols(o, L.g2, L.b2, xo, B, H, P, 1e-5f, s); });
      x = xo;
    }
    float* st = buf("stats", (size_t)B * 2 * HP);
    conv("enc.proj", with16(c1x1(x, HP, proj_w, proj_b, st, B, H, 2 * H, P), proj16));
    float* zp = buf("z_p", (size_t)B * HP);
    if (before_zp) before_zp();
    run("enc.glue", 3.0 * B * HP, 16.0 * B * HP, [&] { launch_zp(st, nz, zp, B, H, P, 0.66666f, s); });
    return zp;
  }

  // flow.reverse of src [B][H][P] (batch stride H*P): Flip, RC(6), Flip,
  // RC(4), ... RC(0) (runtime/models/vits.py, ResidualCouplingBlock reverse).
  // The flips move no data: X holds the reference's tensor with its channel
  // order reversed after an odd number of flips, and such a flow reads its
  // pre conv's half from the top of X with the weight's input channels
  // reversed and subtracts the post conv (rows reversed) from the bottom half
  // (FlowL::rev, set up at finalize).  Each flow's x1 - m is the post conv's
  // subtracting combine where the small-conv kernels run (up to 8192 frames),
  // a separate elementwise launch otherwise; every flow's cond_layer(g) is one
  // stacked gemv up front.  Returns z [B][H][P] in a workspace buffer.
  const float* flow(const float* src, int B, int P, const float* g) {
    hipStream_t s = eng->stream;
    const long long HP = (long long)H * P;
    const long long GW = 2LL * H * kWnLayers;
    float* X = buf("fz0", (size_t)B * HP);
    float* h = buf("fh", (size_t)B * HP);
    float* gv = buf("fgv", (size_t)B * n_flows * GW);
    float* skip = buf("fskip", (size_t)B * HP);
    float* xi = buf("fxi", (size_t)B * 2 * HP);
    float* acts = buf("facts", (size_t)B * HP);
    run("flow.glue", 0.0, 8.0 * B * HP,
        [&] { RVC_HIP(hipMemcpyAsync(X, src, sizeof(float) * B * HP, hipMemcpyDeviceToDevice, s)); });
    run("flow.glue", 2.0 * B * gin * n_flows * GW, 4.0 * (B * gin + (double)(gin + 1 + B) * n_flows * GW),
        [&] { launch_gemv(flow_cond_w, flow_cond_b, g, gin, gv, n_flows * GW, B, (int)(n_flows * GW), gin, s); });
    // Each flow's last res/skip conv, its post conv and the next flow's pre
    // conv run as one launch (flow_tail.hip) where the channel count allows:
    // the next flow's pre reads the half this flow updates.
    const bool tail = flow_tail_supported(H, half) && 4.0 * H * P < 2147483648.0;
    bool pre_done = false;
    for (int fi = n_flows - 1; fi >= 0; --fi) {
      const FlowL& L = flows[fi];
      const long long lo = 0, hi = (long long)half * P;  // channel offsets of X's halves
      const float* x0 = X + (L.rev ? hi : lo);
      float* x1 = X + (L.rev ? lo : hi);
      const float* gf = gv + (long long)fi * GW;
      if (!pre_done) conv("flow.pre", c1x1(x0, HP, L.pre_w, L.pre_b, h, B, half, H, P));
      for (int i = 0; i < kWnLayers; ++i) {
        // in-layer conv + gate: fused into the small-conv kernel's epilogue
        // or the split-K reduce when the conv takes one of those paths (it
        // does at P <= ~8000), a separate elementwise launch otherwise
        ConvLaunch ci = cargs_same(h, HP, P, L.in_w[i], L.in_b[i], xi, 2 * HP, P, B, H, 2 * H, P, kWnKernel, 1,
                                   (kWnKernel - 1) / 2);
        if (conv1d_mfma_fuses_gate(ci)) {
          ci.post = POST_WN_GATE;
          ci.post_g = gf + (long long)i * 2 * H;
          ci.post_gb = n_flows * GW;
          ci.post_H = H;
          ci.g[0].out = acts;
          ci.ob = HP;
          ci.oc = P;
          conv("flow.in", ci);
        } else {
          conv("flow.in", ci);
          run("flow.glue", 0.0, 12.0 * B * HP, [&] {
            launch_wn_gate(xi, 2 * HP, gf + (long long)i * 2 * H, n_flows * GW, acts, B, H, P, s);
          });
        }
        if (tail && i + 1 == kWnLayers) break;  // the last res/skip conv runs in the flow tail
        // res/skip conv as one launch of two output groups over the same
        // input: rows [0, H) accumulate into h (h += rs[:H]), rows [H, 2H)
        // into skip (skip = rs[H:] on the first layer); the last layer has
        // only the skip rows.  Up to 8192 frames the launch runs the
        // whole-reduction 1x1 kernel, which forms h + (sum + b) as the
        // reference does; longer sequences take the one-shot tiled kernel,
        // whose accumulating groups start at (b + h) and add the sum: the
        // same terms in another float32 order.
        const bool has_h = i + 1 < kWnLayers;
        ConvLaunch cr = c1x1(acts, HP, L.rs_w[i], L.rs_b[i], has_h ? h : skip, B, H, H, P);
        cr.w_ld = packed_ld(L.rs_out[i]);
        cr.g[0].combine = has_h || i > 0 ? COMB_ADD : COMB_STORE;
        if (has_h) {
          // group 1 reads its weights at column offset H of rows packed_ld(2H)
          // wide; with H % 4 == 0 its float4 loads (masked to C_out = H rounded
          // up to 4) end inside the row
          RVC_CHECK(H % 4 == 0, "flow: hidden channels must be a multiple of 4");
          cr.n_groups = 2;
          cr.g[1] = cr.g[0];
          cr.g[1].w = L.rs_w[i] + H;
          cr.g[1].bias = L.rs_b[i] + H;
          cr.g[1].out = skip;
          cr.g[1].combine = i == 0 ? COMB_STORE : COMB_ADD;
        }
        conv("flow.rs", cr);
      }
      if (tail) {
        constexpr int kl = kWnLayers - 1;
        FlowTailArgs ta{};
        ta.acts = acts;
        ta.skip = skip;
        ta.w_rs = L.rs_lanes;
        ta.b_rs = L.rs_b[kl];
        ta.w_post = L.post_lanes;
        ta.b_post = L.post_b;
        ta.x1 = x1;
        ta.xb = HP;
        ta.P = P;
        if (fi > 0) {
          const FlowL& N = flows[fi - 1];
          RVC_CHECK(N.rev != L.rev, "flow: the next flow must read the half this one updates");
          ta.w_pre = N.pre_lanes;
          ta.b_pre = N.pre_b;
          ta.h = h;
        }
        const double nxt = fi > 0 ? (double)H * half : 0.0;
        run("flow.tail", 2.0 * B * P * ((double)H * H + (double)half * H + nxt),
            4.0 * ((double)B * P * (2.0 * H + 2.0 * half + (fi > 0 ? H : 0)) + (double)H * H + (double)half * H + nxt),
            [&] { launch_flow_tail(ta, H, B, s); });
        pre_done = fi > 0;
        continue;
      }
      // x1 = x1 - (post(skip) + b), into X's other half (batch stride HP)
      ConvLaunch cp = c1x1(skip, HP, L.post_w, L.post_b, x1, B, H, half, P);
      cp.ob = HP;
      cp.g[0].combine = COMB_SUB;
      if (conv1d_mfma_small_path(cp)) {
        conv("flow.post", cp);
      } else {
        float* m = buf("fm", (size_t)B * half * P);
        conv("flow.post", c1x1(skip, HP, L.post_w, L.post_b, m, B, H, half, P));
        run("flow.glue", (double)B * half * P, 12.0 * B * half * P,
            [&] { launch_sub_inplace_strided(x1, HP, m, (long long)half * P, B, half, P, s); });
      }
    }
    z_name = "fz0";
    if (flows.size() % 2 != 0) {
      // an odd number of flips leaves X reversed: one physical flip
      float* Z = buf("fz1", (size_t)B * HP);
      run("flow.glue", 0.0, 8.0 * B * HP, [&] { launch_flip_channels(X, Z, B, H, P, s); });
      z_name = "fz1";
      return Z;
    }
    return X;
  }

  // enc_p + flow over all P frames (infer_controlled's z)
  const float* enc_flow(const float* phone, const long long* pitch, const float* nz, int B, int P, const float* g,
                        const std::function<void()>& before_zp = {}) {
    return flow(encode(phone, pitch, nz, B, P, before_zp), B, P, g);
  }

  // enc_p over all P frames, then the flow over frames [flow_head, P) only:
  // the reference's partial-synthesis preparation (runtime/models/vits.py:
  // 2416-2476) when flow_head > 0, enc_flow when it is 0.
  const float* enc_flow_from(const float* phone, const long long* pitch, const float* nz, int B, int P, int flow_head,
                             const float* g) {
    float* zp = encode(phone, pitch, nz, B, P);
    if (flow_head == 0) return flow(zp, B, P, g);
    const int Pf = P - flow_head;
    float* crop = buf("z_p_crop", (size_t)B * H * Pf);
    RVC_HIP(hipMemcpy2DAsync(crop, sizeof(float) * Pf, zp + flow_head, sizeof(float) * P, sizeof(float) * Pf,
                             (size_t)B * H, hipMemcpyDeviceToDevice, eng->stream));
    return flow(crop, B, Pf, g);
  }

  // -------------------------------------------------------------- GeneratorNSF
  // Side-stream half of the decoder: the harmonic source, each stage's noise
  // conv (into dN<i>) and cv = cond(g). Ordered after everything already on
  // the engine stream; decode_main() waits for it.
  // g [B][gin] with batch stride gb (0: one speaker for every row), or null
  // for a decoder without the speaker term; seg_off [B][P] (nullable): every
  // frame's phase offset (the reference's seg_offsets) instead of f0's own
  // cumulative phase.
  void decode_prep(const float* g, long long gb, const float* f0, const float* ns, const float* seg_off, int B, int P) {
    // a call that threw between its fork and its join leaves side-stream
    // work behind; finish it before any of its buffers can be reallocated
    if (side) RVC_HIP(hipStreamSynchronize(side));
    if (!side) {
      RVC_HIP(hipStreamCreateWithFlags(&side, hipStreamNonBlocking));
      RVC_HIP(hipEventCreateWithFlags(&forked, hipEventDisableTiming));
      RVC_HIP(hipEventCreateWithFlags(&joined, hipEventDisableTiming));
    }
    const long long N = (long long)P * upp;
    float* har = buf("har", (size_t)B * N);
    dec_har = har;
    float* phase = buf("phase", (size_t)B * P);
    dec_cv = buf("dec_cond", (size_t)B * U);
    dec_noise.assign(n_ups, nullptr);
    {
      long long L = P;
      for (int i = 0; i < n_ups; ++i) {
        L *= rates[i];
        dec_noise[i] = buf("dN" + std::to_string(i), (size_t)B * chans[i] * L);
      }
    }
    RVC_HIP(hipEventRecord(forked, eng->stream));
    RVC_HIP(hipStreamWaitEvent(side, forked, 0));
    hipStream_t s = side;
    run("dec.sine", 20.0 * B * N, 4.0 * B * (2.0 * N + 2.0 * P),
        [&] { launch_sine_source(f0, ns, har, phase, seg_off, B, P, upp, (float)sr, w_lin, b_lin, s); }, s);
    if (g) {
      run("dec.cond", 2.0 * B * U * gin, 4.0 * ((double)B * gin + (double)U * (gin + 1) + (double)B * U),
          [&] { launch_gemv(dcond_w, dcond_b, g, gb, dec_cv, U, B, U, gin, s); }, s);
    } else {
      dec_cv = nullptr;
    }
    char tg[32];
    long long L = P;
    for (int i = 0; i < n_ups; ++i) {
      const int C = chans[i];
      L *= rates[i];
      const long long CL = (long long)C * L;
      if (stages[i].noise_fused) continue;  // formed by the stage's ConvTranspose kernel
      DirectConvArgs d{};
      d.x = har; d.xb = N; d.xc = N;
      d.w = stages[i].nw; d.bias = stages[i].nb;
      d.out = dec_noise[i]; d.ob = CL; d.oc = L;
      d.C_in = 1; d.C_out = C; d.L_in = (int)N;
      d.n_out = (int)((N + 2 * (noise_s[i] / 2) - noise_k[i]) / noise_s[i] + 1);
      RVC_CHECK(d.n_out == L, "noise conv length does not match the upsampled length");
      d.K = noise_k[i]; d.stride = noise_s[i]; d.dil = 1; d.in_off = -(noise_s[i] / 2);
      d.combine = COMB_STORE; d.div = 1.f; d.B = B;
      std::snprintf(tg, sizeof tg, "dec.noise.s%d", i);
      run(tg, 2.0 * B * CL * noise_k[i], 4.0 * B * ((double)N + CL), [&] { launch_conv1d_direct(d, s); }, s);
    }
    RVC_HIP(hipEventRecord(joined, side));
  }

  void decode(const float* z, long long zb, const float* g, long long gb, const float* f0, const float* ns,
              const float* seg_off, int B, int P, float* wave) {
    decode_prep(g, gb, f0, ns, seg_off, B, P);
    decode_main(z, zb, B, P, wave);
  }

  // Engine-stream half: conv_pre (+cv), then per stage ConvTranspose into the
  // stage's noise buffer, the three ResBlocks and their mean, then conv_post.
  void decode_main(const float* z, long long zb, int B, int P, float* wave) {
    hipStream_t s = eng->stream;
    const size_t cap = dec_cap(P);
    float* A = buf("dA", (size_t)B * cap);
    float* T[3];
    float* Y[3];
    for (int j = 0; j < 3; ++j) {
      T[j] = buf("dT" + std::to_string(j), (size_t)B * cap);
      Y[j] = buf("dY" + std::to_string(j), (size_t)B * cap);
    }
    float* pre = buf("dec_pre", (size_t)B * U * P);
    ConvLaunch ca = cargs_same(z, zb, P, dpre_w, dpre_b, pre, (long long)U * P, P, B, H, U, P, 7, 1, 3);
    ca.bias2 = dec_cv;
    ca.bias2b = U;
    RVC_HIP(hipStreamWaitEvent(s, joined, 0));
    conv("dec.pre", ca);
    const float* cur = pre;
    int L = P, c_in = U;
    static const int ks[3] = {3, 7, 11};
    static const int ds[3] = {1, 3, 5};
    char tg[32];
    bool fold_avg = false;
    const float* avg_in[3] = {nullptr, nullptr, nullptr};
    for (int i = 0; i < n_ups; ++i) {
      const int C = chans[i];
      const int Lo = L * rates[i];
      const long long CL = (long long)C * Lo;
      float* X = dec_noise[i];
      // ups: X = ConvTranspose1d(lrelu(cur, 0.1)) + bias + noise_conv(har)
      {
        const int K = kernels[i], st = rates[i], pad = (K - st) / 2;
        const int n_out = (L - 1) * st - 2 * pad + K;
        RVC_CHECK(n_out == Lo, "ConvTranspose output length must equal L * rate");
        std::vector<const float*> ph(stages[i].phases.begin(), stages[i].phases.end());
        std::snprintf(tg, sizeof tg, "dec.ups.s%d", i);
        const StageW& SW = stages[i];
        if (SW.up_all || SW.up_all16) {
          // one output-stationary launch: ConvTranspose + bias + the noise
          // term (computed from har, or read from the side stream's buffer),
          // on fp32 or (precision >= 1) bf16 operands
          ConvTOsLaunch o{};
          o.x = cur; o.xb = (long long)c_in * L; o.L_in = L;
          o.w = SW.up_all; o.w_ld = packed_ld(C); o.bias = SW.up_b;
          o.w16 = SW.up_all16; o.w16_ld = bf16_ld(c_in);
          o.out = X; o.ob = CL; o.oc = Lo; o.L_out = Lo;
          o.B = B; o.C_in = c_in; o.C_out = C; o.K = K; o.S = st; o.pad = pad;
          o.M = (Lo + pad + st - 1) / st;
          o.in_slope = 0.1f;
          o.noise = SW.noise_fused ? nullptr : X;
          o.har = dec_har; o.harb = (long long)P * upp; o.N = (long long)P * upp;
          o.nw = SW.nw; o.nb = SW.nb; o.kn = noise_k[i]; o.ns = noise_s[i]; o.np = noise_s[i] / 2;
          const double nflop = SW.noise_fused ? 2.0 * B * CL * noise_k[i] : 0.0;
          const double nbytes = SW.noise_fused ? 4.0 * B * (double)P * upp : 8.0 * B * CL;
          run(tg, 2.0 * B * (double)c_in * C * K * L + nflop,
              4.0 * B * ((double)c_in * L + CL) + nbytes + 4.0 * c_in * C * K, [&] {
                RVC_CHECK(launch_convt_os(o, s), "dec: no ConvTranspose tile fits stage " + std::to_string(i));
              });
        } else {
          // one grid of `stride` polyphase convolutions accumulating onto the
          // noise conv's output
          run(tg, 2.0 * B * (double)c_in * C * K * L, 4.0 * B * ((double)c_in * L + 2.0 * CL) + 4.0 * c_in * C * K,
              [&] {
                if (!SW.phases16.empty()) {
                  std::vector<const uint16_t*> p16(SW.phases16.begin(), SW.phases16.end());
                  convt_polyphase_bf16(s, cur, (long long)c_in * L, L, p16.data(), bf16_ld(c_in), SW.up_b, X, CL, Lo,
                                       B, c_in, C, L, Lo, K, st, pad, ACT_LEAKY, 0.1f, COMB_ADD);
                } else {
                  convt_polyphase(s, cur, (long long)c_in * L, L, ph.data(), SW.up_b, X, CL, Lo, B, c_in, C, L, Lo, K,
                                  st, pad, ACT_LEAKY, 0.1f, COMB_ADD);
                }
              });
        }
      }
      // three ResBlock1 (k = 3, 7, 11) run side by side: each conv launch
      // carries the same dilation group of all three blocks (k = 11 first, so
      // its longer workgroups are dispatched first); block j keeps its state
      // in T[j]; then A = ((o_3 + o_7) + o_11) / 3.
      std::snprintf(tg, sizeof tg, "dec.rb.s%d", i);
      for (int gi = 0; gi < 3; ++gi) {
        const int d = ds[gi];
        ConvLaunch c1 = cargs_same(nullptr, CL, Lo, nullptr, nullptr, nullptr, CL, Lo, B, C, C, Lo, 1, 1, 0);
        ConvLaunch c2 = c1;
        c1.n_groups = c2.n_groups = 3;
        c1.in_act = ACT_LEAKY; c1.in_slope = 0.1f;
        c1.out_act = ACT_LEAKY; c1.out_slope = 0.1f;
        c2.rb = CL; c2.rc = Lo;
        for (int z = 0; z < 3; ++z) {
          const int j = 2 - z;
          const int k = ks[j];
          const float* src = gi == 0 ? X : T[j];
          ConvGroup& g1 = c1.g[z];
          g1.x = src; g1.w = stages[i].rw[j][0][gi]; g1.bias = stages[i].rb[j][0][gi]; g1.res = nullptr;
          g1.out = Y[j]; g1.K = k; g1.dil = d; g1.in_off = -((k * d - d) / 2);
          ConvGroup& g2 = c2.g[z];
          g2.x = Y[j]; g2.w = stages[i].rw[j][1][gi]; g2.bias = stages[i].rb[j][1][gi]; g2.res = src;
          g2.out = T[j]; g2.K = k; g2.dil = 1; g2.in_off = -((k - 1) / 2);
          g1.out_step = g2.out_step = 1;
          g1.out_off = g2.out_off = 0;
          g1.n_out = g2.n_out = Lo;
          g1.combine = g2.combine = COMB_STORE;
          g1.w16 = stages[i].rw16[j][0][gi];
          g2.w16 = stages[i].rw16[j][1][gi];
        }
        if (c1.g[0].w16) c1.w16_ld = c2.w16_ld = bf16_ld(C);
        conv(tg, c1);
        conv(tg, c2);
      }
      // the last stage's average is formed by conv_post while it stages its
      // input (unless the stage outputs are kept)
      fold_avg = i == n_ups - 1 && !keep_stages;
      if (fold_avg) {
        avg_in[0] = T[0];
        avg_in[1] = T[1];
        avg_in[2] = T[2];
      } else {
        run("dec.avg", 0.0, 16.0 * B * CL, [&] { launch_avg3(A, T[0], T[1], T[2], B * CL, s); });
      }
      if (keep_stages) {
        float* keep = buf("dec_stage" + std::to_string(i), (size_t)B * CL);
        run("dec.keep", 0.0, 8.0 * B * CL, [&] { launch_copy(keep, A, B * CL, s); });
      }
      cur = A;
      L = Lo;
      c_in = C;
    }
    DirectConvArgs p{};
    p.x = cur; p.xb = (long long)c_in * L; p.xc = L;
    if (fold_avg) {
      p.x = avg_in[0];
      p.x2 = avg_in[1];
      p.x3 = avg_in[2];
    }
    p.w = dpost_w; p.bias = nullptr;
    p.out = wave; p.ob = L; p.oc = L;
    p.C_in = c_in; p.C_out = 1; p.L_in = L; p.n_out = L;
    p.K = 7; p.stride = 1; p.dil = 1; p.in_off = -3;
    p.in_act = ACT_LEAKY; p.in_slope = 0.01f;
    p.out_act = ACT_TANH;
    p.combine = COMB_STORE; p.div = 1.f; p.B = B;
    // bytes: every input channel of each input read once (the three ResBlock
    // outputs when the average is folded in), the wave written once
    const double n_in = fold_avg ? 3.0 : 1.0;
    run("dec.post", 2.0 * B * c_in * 7.0 * L, 4.0 * B * (n_in * c_in * L + L) + 4.0 * 7.0 * c_in,
        [&] { launch_conv1d_direct(p, s); });
  }

  void check_ready() const { RVC_CHECK(ready, "synth session not finalized"); }
  void check_BP(long long B, long long P) const {
    RVC_CHECK(B >= 1 && P >= 1 && B <= 4096 && P <= (1 << 22), "invalid batch / frame count");
    RVC_CHECK((size_t)P <= relpos_attention_max_frames(),
              "P exceeds the attention kernel's frame limit (" + std::to_string(relpos_attention_max_frames()) + ")");
  }
};

namespace {
std::mutex g_synth_mu;
std::unordered_map<long long, Synth*> g_synths;
long long g_next_synth = 1;

Synth* synth_from(long long s) {
  std::lock_guard<std::mutex> lk(g_synth_mu);
  auto it = g_synths.find(s);
  return it == g_synths.end() ? nullptr : it->second;
}
}  // namespace

}  // namespace rvc

using namespace rvc;

template <class F>
static int32_t sguard(int64_t sh, F&& body) {
  Synth* s = synth_from(sh);
  if (!s) {
    set_last_error("invalid synth handle");
    return -1;
  }
  try {
    std::lock_guard<std::mutex> lk(s->eng->mu);
    body(*s);
    return 0;
  } catch (const std::exception& ex) {
    set_last_error(ex.what());
    return -1;
  }
}

extern "C" {

int64_t rvc_synth_create(int64_t h) {
  Engine* e = engine_from_handle(h);
  if (!e) {
    set_last_error("invalid engine handle");
    return -1;
  }
  Synth* s = new Synth();
  s->eng = e;
  std::lock_guard<std::mutex> lk(g_synth_mu);
  const long long id = g_next_synth++;
  g_synths[id] = s;
  return id;
}

int32_t rvc_synth_destroy(int64_t sh) {
  Synth* s = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_synth_mu);
    auto it = g_synths.find(sh);
    if (it == g_synths.end()) {
      set_last_error("invalid synth handle");
      return -1;
    }
    s = it->second;
    g_synths.erase(it);
  }
  {
    std::lock_guard<std::mutex> lk(s->eng->mu);
    delete s;
  }
  return 0;
}

int32_t rvc_synth_set_weight(int64_t sh, const char* key, const float* data, const int64_t* shape, int32_t ndim) {
  return sguard(sh, [&](Synth& s) { s.set_weight(key, data, shape, ndim); });
}

int32_t rvc_synth_finalize(int64_t sh, int64_t sr, const int64_t* rates, const int64_t* kernels, int32_t n_ups) {
  return sguard(sh, [&](Synth& s) {
    RVC_CHECK(rates && kernels && n_ups >= 1 && n_ups <= 16 && sr > 0, "finalize: invalid arguments");
    std::vector<int> r(rates, rates + n_ups), k(kernels, kernels + n_ups);
    s.finalize((int)sr, r, k);
  });
}

int32_t rvc_synth_infer_dev(int64_t sh, int64_t phone, int64_t pitch, int64_t nsff0, int64_t sid, int64_t nz,
                            int64_t ns, int64_t B, int64_t P, int64_t wave) {
  return sguard(sh, [&](Synth& s) {
    s.check_ready();
    s.check_BP(B, P);
    Engine& e = *s.eng;
    const float* ph = e.fptr(phone, B * P * s.phone_dim, "infer phone");
    DevBuf& pb = e.get(pitch);
    RVC_CHECK(pb.bytes >= (size_t)(B * P) * 8, "infer pitch: buffer too small (int64 [B,P])");
    const float* f0 = e.fptr(nsff0, B * P, "infer nsff0");
    DevBuf& sb = e.get(sid);
    RVC_CHECK(sb.bytes >= (size_t)B * 8, "infer sid: buffer too small (int64 [B])");
    const float* nzp = e.fptr(nz, B * s.H * P, "infer nz");
    const float* nsp = e.fptr(ns, B * P * s.upp, "infer ns");
    float* wv = e.fptr(wave, B * P * s.upp, "infer wave");
    float* g = s.buf("g", (size_t)B * s.gin);
    s.begin_ids();
    s.speaker(static_cast<const long long*>(sb.ptr), (int)B, g);
    s.decode_prep(g, s.gin, f0, nsp, nullptr, (int)B, (int)P);
    const float* z = s.enc_flow(ph, static_cast<const long long*>(pb.ptr), nzp, (int)B, (int)P, g);
    s.decode_main(z, (long long)s.H * P, (int)B, (int)P, wv);
    s.close_span();
    s.fetch_ids();
    e.sync();
    s.collect_timing();
    s.check_ids();
  });
}

namespace {
void check_ids_host(const Synth& s, const int64_t* pitch, const int64_t* sid, long long B, long long P);
}  // namespace

int64_t rvc_synth_submit(int64_t sh, const float* phone, int64_t phone_buf, const int64_t* pitch,
                         const float* nsff0, const int64_t* sid, const float* nz, const float* ns, int64_t B,
                         int64_t P) {
  int64_t ticket = -1;
  const int32_t rc = sguard(sh, [&](Synth& s) {
    s.check_ready();
    s.check_BP(B, P);
    RVC_CHECK((phone != nullptr) != (phone_buf != 0), "submit: pass exactly one of phone and phone_buf");
    RVC_CHECK(pitch && nsff0 && sid && nz && ns, "submit: null pointer");
    check_ids_host(s, pitch, sid, B, P);
    hipStream_t st = s.eng->stream;
    const long long N = P * s.upp;
    const float* d_ph = nullptr;
    if (phone_buf != 0) {
      d_ph = s.eng->fptr(phone_buf, B * P * s.phone_dim, "submit phone_buf");
    } else {
      float* d = s.buf("in_phone", (size_t)(B * P * s.phone_dim));
      RVC_HIP(hipMemcpyAsync(d, phone, sizeof(float) * B * P * s.phone_dim, hipMemcpyHostToDevice, st));
      d_ph = d;
    }
    float* d_pitch = s.buf("in_pitch", (size_t)(B * P * 2));
    float* d_f0 = s.buf("in_f0", (size_t)(B * P));
    float* d_sid = s.buf("in_sid", (size_t)(B * 2));
    float* d_nz = s.buf("in_nz", (size_t)(B * s.H * P));
    float* d_ns = s.buf("in_ns", (size_t)(B * N));
    float* d_w = s.buf("out_wave", (size_t)(B * N));
    s.pending_room();
    // as in rvc_synth_infer: nz, f0 and the NSF noise upload behind the encoder
    RVC_HIP(hipMemcpyAsync(d_pitch, pitch, 8 * B * P, hipMemcpyHostToDevice, st));
    RVC_HIP(hipMemcpyAsync(d_sid, sid, 8 * B, hipMemcpyHostToDevice, st));
    float* g = s.buf("g", (size_t)B * s.gin);
    s.speaker(reinterpret_cast<const long long*>(d_sid), (int)B, g);
    const float* z = s.enc_flow(d_ph, reinterpret_cast<const long long*>(d_pitch), d_nz, (int)B, (int)P, g, [&] {
      RVC_HIP(hipMemcpyAsync(d_nz, nz, sizeof(float) * B * s.H * P, hipMemcpyHostToDevice, st));
      RVC_HIP(hipMemcpyAsync(d_f0, nsff0, sizeof(float) * B * P, hipMemcpyHostToDevice, st));
      RVC_HIP(hipMemcpyAsync(d_ns, ns, sizeof(float) * B * N, hipMemcpyHostToDevice, st));
      s.decode_prep(g, s.gin, d_f0, d_ns, nullptr, (int)B, (int)P);
    });
    s.decode_main(z, (long long)s.H * P, (int)B, (int)P, d_w);
    s.close_span();
    Synth::Pending& slot = s.pending_slot(B * N);
    RVC_HIP(hipMemcpyAsync(slot.host, d_w, sizeof(float) * B * N, hipMemcpyDeviceToHost, st));
    RVC_HIP(hipEventRecord(slot.done, st));
    ticket = slot.id;
  });
  return rc == 0 ? ticket : -1;
}

int32_t rvc_synth_collect(int64_t sh, int64_t ticket, float* wave) {
  return sguard(sh, [&](Synth& s) {
    RVC_CHECK(wave != nullptr, "collect: null pointer");
    Synth::Pending& p = s.pending_find(ticket);
    const hipError_t e = hipEventSynchronize(p.done);
    const long long n = p.n;
    if (e == hipSuccess) std::memcpy(wave, p.host, sizeof(float) * n);
    p.id = 0;  // the slot is free again, whatever the outcome
    RVC_HIP(e);
  });
}

int32_t rvc_synth_abort(int64_t sh, int64_t ticket) {
  return sguard(sh, [&](Synth& s) {
    Synth::Pending& p = s.pending_find(ticket);
    const hipError_t e = hipEventSynchronize(p.done);
    p.id = 0;
    RVC_HIP(e);
  });
}

namespace {
void check_ids_host(const Synth& s, const int64_t* pitch, const int64_t* sid, long long B, long long P) {
  for (long long i = 0; i < B * P; ++i)
    RVC_CHECK(pitch[i] >= -s.pitch_rows && pitch[i] < s.pitch_rows, "infer: pitch id out of range");
  for (long long i = 0; i < B; ++i) RVC_CHECK(sid[i] >= -s.n_spk && sid[i] < s.n_spk, "infer: sid out of range");
}
}  // namespace

int32_t rvc_synth_infer(int64_t sh, const float* phone, const int64_t* pitch, const float* nsff0, const int64_t* sid,
                        const float* nz, const float* ns, int64_t B, int64_t P, float* wave) {
  return sguard(sh, [&](Synth& s) {
    s.check_ready();
    s.check_BP(B, P);
    RVC_CHECK(phone && pitch && nsff0 && sid && nz && ns && wave, "infer: null pointer");
    check_ids_host(s, pitch, sid, B, P);
    hipStream_t st = s.eng->stream;
    const long long N = P * s.upp;
    float* d_ph = s.buf("in_phone", (size_t)(B * P * s.phone_dim));
    float* d_pitch = s.buf("in_pitch", (size_t)(B * P * 2));
    float* d_f0 = s.buf("in_f0", (size_t)(B * P));
    float* d_sid = s.buf("in_sid", (size_t)(B * 2));
    float* d_nz = s.buf("in_nz", (size_t)(B * s.H * P));
    float* d_ns = s.buf("in_ns", (size_t)(B * N));
    float* d_w = s.buf("out_wave", (size_t)(B * N));
    // The encoder needs only phone, pitch and sid: they go first, the
    // encoder is queued, and the host then uploads nz, f0 and the NSF noise
    // while the GPU runs it (pageable copies return once staged, in stream
    // order before z_p and the decoder's source that read them).
    RVC_HIP(hipMemcpyAsync(d_ph, phone, sizeof(float) * B * P * s.phone_dim, hipMemcpyHostToDevice, st));
    RVC_HIP(hipMemcpyAsync(d_pitch, pitch, 8 * B * P, hipMemcpyHostToDevice, st));
    RVC_HIP(hipMemcpyAsync(d_sid, sid, 8 * B, hipMemcpyHostToDevice, st));
    float* g = s.buf("g", (size_t)B * s.gin);
    s.speaker(reinterpret_cast<const long long*>(d_sid), (int)B, g);
    const float* z = s.enc_flow(d_ph, reinterpret_cast<const long long*>(d_pitch), d_nz, (int)B, (int)P, g, [&] {
      RVC_HIP(hipMemcpyAsync(d_nz, nz, sizeof(float) * B * s.H * P, hipMemcpyHostToDevice, st));
      RVC_HIP(hipMemcpyAsync(d_f0, nsff0, sizeof(float) * B * P, hipMemcpyHostToDevice, st));
      RVC_HIP(hipMemcpyAsync(d_ns, ns, sizeof(float) * B * N, hipMemcpyHostToDevice, st));
      s.decode_prep(g, s.gin, d_f0, d_ns, nullptr, (int)B, (int)P);
    });
    s.decode_main(z, (long long)s.H * P, (int)B, (int)P, d_w);
    s.close_span();
    RVC_HIP(hipMemcpyAsync(wave, d_w, sizeof(float) * B * N, hipMemcpyDeviceToHost, st));
    RVC_HIP(hipStreamSynchronize(st));
    s.collect_timing();
  });
}

int32_t rvc_synth_prep(int64_t sh, const float* phone, const int64_t* pitch, const float* nsff0, const int64_t* sid,
                       const float* nz, int64_t B, int64_t P, int64_t flow_head, float* z_out, float* g_out,
                       float* phase_out) {
  return sguard(sh, [&](Synth& s) {
    s.check_ready();
    s.check_BP(B, P);
    RVC_CHECK(phone && pitch && sid && nz && z_out, "prep: null pointer");
    RVC_CHECK(flow_head >= 0 && flow_head < P, "prep: flow_head must be in [0, P)");
    RVC_CHECK(!phase_out || nsff0, "prep: phase offsets need nsff0");
    check_ids_host(s, pitch, sid, B, P);
    hipStream_t st = s.eng->stream;
    const long long Pf = P - flow_head;
    float* d_ph = s.buf("in_phone", (size_t)(B * P * s.phone_dim));
    float* d_pitch = s.buf("in_pitch", (size_t)(B * P * 2));
    float* d_sid = s.buf("in_sid", (size_t)(B * 2));
    float* d_nz = s.buf("in_nz", (size_t)(B * s.H * P));
    RVC_HIP(hipMemcpyAsync(d_ph, phone, sizeof(float) * B * P * s.phone_dim, hipMemcpyHostToDevice, st));
    RVC_HIP(hipMemcpyAsync(d_pitch, pitch, 8 * B * P, hipMemcpyHostToDevice, st));
    RVC_HIP(hipMemcpyAsync(d_sid, sid, 8 * B, hipMemcpyHostToDevice, st));
    RVC_HIP(hipMemcpyAsync(d_nz, nz, sizeof(float) * B * s.H * P, hipMemcpyHostToDevice, st));
    float* g = s.buf("g", (size_t)B * s.gin);
    s.speaker(reinterpret_cast<const long long*>(d_sid), (int)B, g);
    const float* z = s.enc_flow_from(d_ph, reinterpret_cast<const long long*>(d_pitch), d_nz, (int)B, (int)P,
                                     (int)flow_head, g);
    s.close_span();  // the phase scan below is no part of the flow's timing
    if (phase_out) {
      float* d_f0 = s.buf("in_f0", (size_t)(B * P));
      float* d_phase = s.buf("prep_phase", (size_t)(B * P));
      RVC_HIP(hipMemcpyAsync(d_f0, nsff0, sizeof(float) * B * P, hipMemcpyHostToDevice, st));
      launch_sine_phase(d_f0, d_phase, (int)B, (int)P, s.upp, (float)s.sr, 0, st);
      RVC_HIP(hipMemcpyAsync(phase_out, d_phase, sizeof(float) * B * P, hipMemcpyDeviceToHost, st));
    }
    RVC_HIP(hipMemcpyAsync(z_out, z, sizeof(float) * B * s.H * Pf, hipMemcpyDeviceToHost, st));
    if (g_out) RVC_HIP(hipMemcpyAsync(g_out, g, sizeof(float) * B * s.gin, hipMemcpyDeviceToHost, st));
    RVC_HIP(hipStreamSynchronize(st));
    s.collect_timing();
  });
}

int32_t rvc_synth_phase_offsets(int64_t sh, const float* nsff0, int64_t B, int64_t P, float* out) {
  return sguard(sh, [&](Synth& s) {
    s.check_ready();
    s.check_BP(B, P);
    RVC_CHECK(nsff0 && out, "phase_offsets: null pointer");
    hipStream_t st = s.eng->stream;
    float* d_f0 = s.buf("in_f0", (size_t)(B * P));
    float* d_phase = s.buf("prep_phase", (size_t)(B * P));
    RVC_HIP(hipMemcpyAsync(d_f0, nsff0, sizeof(float) * B * P, hipMemcpyHostToDevice, st));
    launch_sine_phase(d_f0, d_phase, (int)B, (int)P, s.upp, (float)s.sr, 0, st);
    RVC_HIP(hipMemcpyAsync(out, d_phase, sizeof(float) * B * P, hipMemcpyDeviceToHost, st));
    RVC_HIP(hipStreamSynchronize(st));
  });
}

int32_t rvc_synth_decode_dev(int64_t sh, int64_t z, int64_t f0, int64_t g, int64_t ns, int64_t B, int64_t P,
                             int64_t wave) {
  return sguard(sh, [&](Synth& s) {
    s.check_ready();
    s.check_BP(B, P);
    Engine& e = *s.eng;
    const float* zp = e.fptr(z, B * s.H * P, "decode z");
    const float* fp = e.fptr(f0, B * P, "decode f0");
    const float* gp = e.fptr(g, B * s.gin, "decode g");
    const float* np_ = e.fptr(ns, B * P * s.upp, "decode ns");
    float* wv = e.fptr(wave, B * P * s.upp, "decode wave");
    s.decode(zp, (long long)s.H * P, gp, s.gin, fp, np_, nullptr, (int)B, (int)P, wv);
    s.close_span();
    e.sync();
    s.collect_timing();
  });
}

int32_t rvc_synth_decode(int64_t sh, const float* z, const float* f0, const float* g, const float* ns, int64_t B,
                         int64_t P, float* wave) {
  return sguard(sh, [&](Synth& s) {
    s.check_ready();
    s.check_BP(B, P);
    RVC_CHECK(z && f0 && g && ns && wave, "decode: null pointer");
    hipStream_t st = s.eng->stream;
    const long long N = P * s.upp;
    float* d_z = s.buf("in_z", (size_t)(B * s.H * P));
    float* d_f0 = s.buf("in_f0", (size_t)(B * P));
    float* d_g = s.buf("in_g", (size_t)(B * s.gin));
    float* d_ns = s.buf("in_ns", (size_t)(B * N));
    float* d_w = s.buf("out_wave", (size_t)(B * N));
    RVC_HIP(hipMemcpyAsync(d_z, z, sizeof(float) * B * s.H * P, hipMemcpyHostToDevice, st));
    RVC_HIP(hipMemcpyAsync(d_f0, f0, sizeof(float) * B * P, hipMemcpyHostToDevice, st));
    RVC_HIP(hipMemcpyAsync(d_g, g, sizeof(float) * B * s.gin, hipMemcpyHostToDevice, st));
    RVC_HIP(hipMemcpyAsync(d_ns, ns, sizeof(float) * B * N, hipMemcpyHostToDevice, st));
    s.decode(d_z, (long long)s.H * P, d_g, s.gin, d_f0, d_ns, nullptr, (int)B, (int)P, d_w);
    s.close_span();
    RVC_HIP(hipMemcpyAsync(wave, d_w, sizeof(float) * B * N, hipMemcpyDeviceToHost, st));
    RVC_HIP(hipStreamSynchronize(st));
    s.collect_timing();
  });
}

int32_t rvc_synth_decode_chunks(int64_t sh, int64_t n, const float* const* z, const float* const* f0,
                                const float* const* ns, const float* const* off, const int64_t* P, const float* g,
                                float* const* wave) {
  return sguard(sh, [&](Synth& s) {
    s.check_ready();
    RVC_CHECK(n >= 1 && n <= 4096, "decode_chunks: chunk count must be in [1, 4096]");
    RVC_CHECK(z && f0 && ns && P && wave, "decode_chunks: null pointer");
    for (long long i = 0; i < n; ++i) {
      RVC_CHECK(z[i] && f0[i] && ns[i] && wave[i], "decode_chunks: null pointer in chunk " + std::to_string(i));
      s.check_BP(1, P[i]);
    }
    // Chunks of one length, with or without phase offsets, run as one batch;
    // the batches follow each other on the stream with no synchronisation in
    // between.  Batch rows keep the chunks' order, and a batch's kernels
    // and tiles depend on (P, rows) only, so every chunk's result equals
    // its own single-chunk decode.
    struct Group {
      long long P;
      bool off;
      std::vector<long long> idx;
    };
    std::vector<Group> groups;
    for (long long i = 0; i < n; ++i) {
      const bool has_off = off && off[i];
      auto it = std::find_if(groups.begin(), groups.end(),
                             [&](const Group& gr) { return gr.P == P[i] && gr.off == has_off; });
      if (it == groups.end()) {
        groups.push_back(Group{P[i], has_off, {}});
        it = groups.end() - 1;
      }
      it->idx.push_back(i);
    }
    // largest batch first, so the workspace is sized once
    std::stable_sort(groups.begin(), groups.end(), [](const Group& x, const Group& y) {
      return x.P * (long long)x.idx.size() > y.P * (long long)y.idx.size();
    });
    size_t maxBP = 0;
    for (const Group& gr : groups) maxBP = std::max(maxBP, (size_t)(gr.P * (long long)gr.idx.size()));
    hipStream_t st = s.eng->stream;
    float* d_z = s.buf("in_z", maxBP * s.H);
    float* d_f0 = s.buf("in_f0", maxBP);
    float* d_off = s.buf("in_off", maxBP);
    float* d_ns = s.buf("in_ns", maxBP * s.upp);
    float* d_w = s.buf("out_wave", maxBP * s.upp);
    float* d_g = nullptr;
    if (g) {
      d_g = s.buf("in_g", (size_t)s.gin);
      RVC_HIP(hipMemcpyAsync(d_g, g, sizeof(float) * s.gin, hipMemcpyHostToDevice, st));
    }
    for (const Group& gr : groups) {
      const long long Pg = gr.P, N = Pg * s.upp;
      const int Bg = (int)gr.idx.size();
      for (int r = 0; r < Bg; ++r) {
        const long long i = gr.idx[r];
        RVC_HIP(hipMemcpyAsync(d_z + r * s.H * Pg, z[i], sizeof(float) * s.H * Pg, hipMemcpyHostToDevice, st));
        RVC_HIP(hipMemcpyAsync(d_f0 + r * Pg, f0[i], sizeof(float) * Pg, hipMemcpyHostToDevice, st));
        RVC_HIP(hipMemcpyAsync(d_ns + r * N, ns[i], sizeof(float) * N, hipMemcpyHostToDevice, st));
        if (gr.off) RVC_HIP(hipMemcpyAsync(d_off + r * Pg, off[i], sizeof(float) * Pg, hipMemcpyHostToDevice, st));
      }
      s.decode(d_z, (long long)s.H * Pg, d_g, 0, d_f0, d_ns, gr.off ? d_off : nullptr, Bg, (int)Pg, d_w);
      for (int r = 0; r < Bg; ++r)
        RVC_HIP(hipMemcpyAsync(wave[gr.idx[r]], d_w + r * N, sizeof(float) * N, hipMemcpyDeviceToHost, st));
    }
    s.close_span();
    RVC_HIP(hipStreamSynchronize(st));
    s.collect_timing();
  });
}

int32_t rvc_synth_read(int64_t sh, const char* name, float* dst, int64_t n) {
  return sguard(sh, [&](Synth& s) {
    RVC_CHECK(name && dst && n >= 0, "read: invalid arguments");
    s.read(std::strcmp(name, "z") == 0 ? s.z_name : std::string(name), dst, n);
  });
}

int32_t rvc_synth_set_precision(int64_t sh, int32_t mode) {
  return sguard(sh, [&](Synth& s) {
    RVC_CHECK(!s.ready, "set_precision: the session is already finalized");
    RVC_CHECK(mode >= 0 && mode <= 2, "set_precision: mode must be 0 (fp32), 1 (bf16 ups + enc_p) or 2 (1 + ResBlocks)");
    s.precision = mode;
  });
}

int32_t rvc_synth_set_debug(int64_t sh, int32_t keep_stages) {
  return sguard(sh, [&](Synth& s) { s.keep_stages = keep_stages != 0; });
}

int32_t rvc_synth_set_timing(int64_t sh, const char* tag) {
  return sguard(sh, [&](Synth& s) { s.set_timing(tag); });
}

int32_t rvc_synth_get_timing(int64_t sh, double* total_ms, int64_t* launches, double* flops, double* bytes) {
  return sguard(sh, [&](Synth& s) {
    if (total_ms) *total_ms = s.t_ms;
    if (launches) *launches = s.t_n;
    if (flops) *flops = s.t_flops;
    if (bytes) *bytes = s.t_bytes;
  });
}

}  // extern "C"
