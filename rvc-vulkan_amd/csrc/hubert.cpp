// Device-resident HuBERT-base encoder session (rvc_hubert_* exports).
//
// Runs HubertEncoder.encode (runtime/models/hubert.py:564-591) on one stream:
//   feature extractor  :658-697   conv0 (1 -> C, k10 s5, vector ALU) ->
//                                 GroupNorm(C groups) + GELU -> 6 strided MFMA
//                                 convs with GELU fused in the epilogue
//   feature projection :775-802   channel LayerNorm -> 1x1 conv (+ bias)
//   encoder entry      :838-858, :928-940  grouped k128 positional conv as
//                                 tap blocks of <= 11 taps accumulated in
//                                 place (all 16 channel groups per launch),
//                                 h + gelu(pos), channel LayerNorm
//   12 post-LN layers  :1262-1338, :1401-1451  stacked q/k/v 1x1 conv,
//                                 fused attention (12 heads x 64), out 1x1 conv
//                                 + residual, LN, FFN 1x1 convs with GELU
//                                 fused, + residual, LN
// Activations stay channel-major [B][C][L]; the result is transposed to the
// reference's [B, L, C] on the device.  GELU is the reference's A&S erf form.
#include <cmath>
#include <cstring>

#include "../../include/rvc_hip.h"
#include "session.h"

namespace rvc {

struct Hubert : SessionBase {
  static constexpr int kHeads = 12;        // runtime/models/hubert.py:1326
  static constexpr int kTapBlock = kConvTapsMax;
  int C = 0, H = 0, F = 0, n_layers = 0, n_conv = 0, D = 0, final_dim = 0;
  int pos_k = 0, pos_groups = 0, cpg = 0;
  std::vector<int> conv_k, conv_s;
  bool keep = false;

  float* conv0_w = nullptr;               // [C][1][k0] (vector-ALU conv)
  std::vector<float*> conv_w;             // packed, layers 1..n_conv-1
  float *gn_g = nullptr, *gn_b = nullptr;
  float *fp_ln_g = nullptr, *fp_ln_b = nullptr, *fp_w = nullptr, *fp_b = nullptr;
  std::vector<float*> pos_w;              // per tap block: pos_groups packed slabs [Kb][cpg][ld]
  std::vector<int> pos_k0, pos_kb;
  float* pos_wl = nullptr;                // [groups][K][cpg in][cpg out] for the one-launch kernel
  float *pos_b = nullptr, *enc_ln_g = nullptr, *enc_ln_b = nullptr;
  struct Layer {
    float *wqkv, *bqkv, *wo, *bo, *ln1_g, *ln1_b, *wi, *bi, *wf, *bf, *ln2_g, *ln2_b;
    // the LayerNorm in front folded in, W diag(g) and b + W beta: the FFN
    // input GEMM with LN1, the q/k/v GEMM with the previous layer's LN2
    // (null for layer 0, whose input the encoder's LayerNorm launch forms)
    float *wi_ln, *bi_ln, *wqkv_ln, *bqkv_ln;
  };
  std::vector<Layer> layers;
  float *final_w = nullptr, *final_b = nullptr;

  const HostT& Wn(const std::string& a, const std::string& b) const { return has(a) ? W(a) : W(b); }

  float* upload_linear(const std::string& key, long long O, long long I) {
    const HostT& t = W(key + ".weight");
    check_shape(key + ".weight", t.shape, {O, I});
    return upload(pack(t.data, O, I, 1));
  }

  // A linear layer [O][I] (+ bias [O]) behind a LayerNorm with affine g, beta
  // over its I inputs, folded: W'[o][i] = W[o][i] * g[i] (float32 product),
  // b'[o] = b[o] + sum_i W[o][i] * beta[i] (float64 sum, rounded once).
  // Uploads the packed W' and returns b' uploaded through *bias.
  float* upload_folded(const std::vector<float>& w, const std::vector<float>& b, const std::vector<float>& g,
                       const std::vector<float>& beta, long long O, long long I, float** bias) {
    std::vector<float> wf(w.size()), bf(O);
    for (long long o = 0; o < O; ++o) {
      double acc = 0.0;
      for (long long i = 0; i < I; ++i) {
        wf[o * I + i] = w[o * I + i] * g[i];
        acc += (double)w[o * I + i] * beta[i];
      }
      bf[o] = (float)((double)b[o] + acc);
    }
    *bias = upload(bf);
    return upload(pack(wf, O, I, 1));
  }

  void finalize() {
    RVC_CHECK(!ready, "hubert session already finalized");
    while (has("feature_extractor.conv_layers." + std::to_string(n_conv) + ".conv.weight")) ++n_conv;
    RVC_CHECK(n_conv >= 2, "hubert: need the feature extractor conv layers");
    while (has("encoder.layers." + std::to_string(n_layers) + ".attention.q_proj.weight")) ++n_layers;
    const HostT& c0 = W("feature_extractor.conv_layers.0.conv.weight");
    RVC_CHECK(c0.shape.size() == 3 && c0.shape[1] == 1, "conv layer 0 must be [C, 1, k]");
    C = (int)c0.shape[0];
    const HostT& fp = W("feature_projection.projection.weight");
    RVC_CHECK(fp.shape.size() == 2 && fp.shape[1] == C, "feature_projection.projection.weight must be [H, C]");
    H = (int)fp.shape[0];
    RVC_CHECK(H % kHeads == 0, "hidden size must split into 12 heads");
    D = H / kHeads;
    RVC_CHECK(D <= 128, "head dim must be <= 128");

    // ---- feature extractor (strides 5, 2, 2, ...: runtime/models/hubert.py:680)
    conv0_w = upload(c0.data);
    conv_k.push_back((int)c0.shape[2]);
    conv_s.push_back(5);
    for (int i = 1; i < n_conv; ++i) {
      const std::string k = "feature_extractor.conv_layers." + std::to_string(i) + ".conv.weight";
      const HostT& t = W(k);
      RVC_CHECK(t.shape.size() == 3 && t.shape[0] == C && t.shape[1] == C, k + " must be [C, C, k]");
      const int K = (int)t.shape[2];
      RVC_CHECK(conv1d_mfma_supported(K, 1), k + ": taps outside the MFMA path");
      conv_k.push_back(K);
      conv_s.push_back(2);
      conv_w.push_back(upload(pack(t.data, C, C, K)));
    }
    gn_g = upload_vec("feature_extractor.conv_layers.0.layer_norm.weight", C);
    gn_b = upload_vec("feature_extractor.conv_layers.0.layer_norm.bias", C);
    fp_ln_g = upload_vec("feature_projection.layer_norm.weight", C);
    fp_ln_b = upload_vec("feature_projection.layer_norm.bias", C);
    fp_w = upload_linear("feature_projection.projection", H, C);
    fp_b = upload_vec("feature_projection.projection.bias", H);

    // ---- positional conv: weight norm over dims (0, 1) per tap
    //      W = g * (v / ||v[:, :, k]||)  (runtime/models/hubert.py:510-522)
    const HostT& v = Wn("encoder.pos_conv_embed.conv.weight_v",
                        "encoder.pos_conv_embed.conv.parametrizations.weight.original1");
    const HostT& g = Wn("encoder.pos_conv_embed.conv.weight_g",
                        "encoder.pos_conv_embed.conv.parametrizations.weight.original0");
    RVC_CHECK(v.shape.size() == 3 && v.shape[0] == H, "pos conv weight_v must be [H, H/groups, k]");
    cpg = (int)v.shape[1];
    pos_k = (int)v.shape[2];
    RVC_CHECK(cpg >= 1 && H % cpg == 0, "pos conv: channels per group must divide H");
    pos_groups = H / cpg;
    RVC_CHECK(pos_groups <= kMaxConvGroups, "pos conv: too many groups for one launch");
    RVC_CHECK((long long)g.data.size() == pos_k, "pos conv weight_g must hold one scale per tap");
    std::vector<float> wpos(v.data.size());
    for (int k = 0; k < pos_k; ++k) {
      double s = 0;
      for (long long i = 0; i < (long long)H * cpg; ++i) {
        const double x = v.data[i * pos_k + k];
        s += x * x;
      }
      const float nrm = (float)std::sqrt(s);
      for (long long i = 0; i < (long long)H * cpg; ++i)
        wpos[i * pos_k + k] = g.data[k] * (v.data[i * pos_k + k] / nrm);
    }
    if (posconv_supported(cpg, pos_k, pos_k / 2)) {
      std::vector<float> wl((size_t)pos_groups * pos_k * cpg * cpg);
      for (int gi = 0; gi < pos_groups; ++gi)
        for (int k = 0; k < pos_k; ++k)
          for (int ci = 0; ci < cpg; ++ci)
            for (int co = 0; co < cpg; ++co)
              wl[(((size_t)gi * pos_k + k) * cpg + ci) * cpg + co] =
                  wpos[(((size_t)gi * cpg + co) * cpg + ci) * pos_k + k];
      pos_wl = upload(wl);
    }
    const int ld = packed_ld(cpg);
    for (int k0 = 0; pos_wl == nullptr && k0 < pos_k; k0 += kTapBlock) {
      const int kb = std::min(kTapBlock, pos_k - k0);
      std::vector<float> blk((size_t)pos_groups * kb * cpg * ld, 0.f);
      for (int gi = 0; gi < pos_groups; ++gi) {
        float* dst = blk.data() + (size_t)gi * kb * cpg * ld;
        for (int co = 0; co < cpg; ++co)
          for (int ci = 0; ci < cpg; ++ci)
            for (int k = 0; k < kb; ++k)
              dst[((size_t)k * cpg + ci) * ld + co] = wpos[(((size_t)gi * cpg + co) * cpg + ci) * pos_k + k0 + k];
      }
      pos_w.push_back(upload(blk));
      pos_k0.push_back(k0);
      pos_kb.push_back(kb);
    }
    pos_b = upload_vec("encoder.pos_conv_embed.conv.bias", H);
    enc_ln_g = upload_vec("encoder.layer_norm.weight", H);
    enc_ln_b = upload_vec("encoder.layer_norm.bias", H);

    // ---- transformer layers
    F = (int)W("encoder.layers.0.feed_forward.intermediate_dense.weight").shape[0];
    for (int i = 0; i < n_layers; ++i) {
      const std::string p = "encoder.layers." + std::to_string(i) + ".";
      Layer L{};
      std::vector<float> qkv, bqkv;
      for (const char* nm : {"q_proj", "k_proj", "v_proj"}) {
        const HostT& t = W(p + "attention." + nm + ".weight");
        check_shape(p + "attention." + nm + ".weight", t.shape, {H, H});
        qkv.insert(qkv.end(), t.data.begin(), t.data.end());
        const HostT& b = W(p + "attention." + nm + ".bias");
        RVC_CHECK((int)b.data.size() == H, p + "attention bias size");
        bqkv.insert(bqkv.end(), b.data.begin(), b.data.end());
      }
      L.wqkv = upload(pack(qkv, 3 * H, H, 1));
      L.bqkv = upload(bqkv);
      if (i > 0) {
        const std::string q = "encoder.layers." + std::to_string(i - 1) + ".final_layer_norm.";
        L.wqkv_ln = upload_folded(qkv, bqkv, W(q + "weight").data, W(q + "bias").data, 3 * H, H, &L.bqkv_ln);
      }
      L.wo = upload_linear(p + "attention.out_proj", H, H);
      L.bo = upload_vec(p + "attention.out_proj.bias", H);
      L.ln1_g = upload_vec(p + "layer_norm.weight", H);
      L.ln1_b = upload_vec(p + "layer_norm.bias", H);
      L.wi = upload_linear(p + "feed_forward.intermediate_dense", F, H);
      L.bi = upload_vec(p + "feed_forward.intermediate_dense.bias", F);
      L.wi_ln = upload_folded(W(p + "feed_forward.intermediate_dense.weight").data,
                              W(p + "feed_forward.intermediate_dense.bias").data, W(p + "layer_norm.weight").data,
                              W(p + "layer_norm.bias").data, F, H, &L.bi_ln);
      L.wf = upload_linear(p + "feed_forward.output_dense", H, F);
      L.bf = upload_vec(p + "feed_forward.output_dense.bias", H);
      L.ln2_g = upload_vec(p + "final_layer_norm.weight", H);
      L.ln2_b = upload_vec(p + "final_layer_norm.bias", H);
      layers.push_back(L);
    }
    if (has("final_proj.weight")) {
      final_dim = (int)W("final_proj.weight").shape[0];
      final_w = upload_linear("final_proj", final_dim, H);
      final_b = upload_vec("final_proj.bias", final_dim);
    }
    host.clear();
    ready = true;
  }

  long long frames(long long T) const {
    long long L = T;
    for (size_t i = 0; i < conv_k.size(); ++i) L = L < conv_k[i] ? 0 : (L - conv_k[i]) / conv_s[i] + 1;
    return L;
  }

  void check_args(long long B, long long T, int version) const {
    RVC_CHECK(ready, "hubert session not finalized");
    RVC_CHECK(B >= 1 && B <= 1024 && T >= 1, "invalid batch / sample count");
    RVC_CHECK(version == 1 || version == 2, "version must be 1 or 2");
    RVC_CHECK(version == 2 || (final_w && n_layers >= 9), "version 1 needs final_proj and 9 layers");
    RVC_CHECK(frames(T) >= 1, "input shorter than the feature extractor's receptive field");
    RVC_CHECK((size_t)frames(T) <= relpos_attention_max_frames(), "too many frames");
  }

  int out_dim(int version) const { return version == 1 ? final_dim : H; }

  // x [B][T] -> out [B][L][out_dim(version)]
  void encode(const float* x, int B, long long T, int version, float* out) {
    hipStream_t s = eng->stream;
    // ---- feature extractor
    long long L = (T - conv_k[0]) / conv_s[0] + 1;
    float* a = buf("conv_a", (size_t)B * C * L);
    float* c = buf("conv_b", (size_t)B * C * L);
    {
      DirectConvArgs d{};
      d.x = x; d.xb = T; d.xc = T;
      d.w = conv0_w; d.bias = nullptr;
      d.out = a; d.ob = (long long)C * L; d.oc = L;
      d.C_in = 1; d.C_out = C; d.L_in = (int)T; d.n_out = (int)L;
      d.K = conv_k[0]; d.stride = conv_s[0]; d.dil = 1; d.in_off = 0;
      d.combine = COMB_STORE; d.div = 1.f; d.B = B;
      run("hub.conv0", 2.0 * B * C * conv_k[0] * (double)L, 4.0 * B * ((double)T + (double)C * L),
          [&] { launch_conv1d_direct(d, s); });
    }
    run("hub.gn", 10.0 * B * C * L, 12.0 * B * C * L,
        [&] { launch_groupnorm_rows_act(a, gn_g, gn_b, c, B, C, L, 1e-5f, ACT_GELU, s); });
    std::swap(a, c);
    for (int i = 1; i < n_conv; ++i) {
      const long long Lo = (L - conv_k[i]) / conv_s[i] + 1;
      ConvLaunch cl = cargs(a, (long long)C * L, L, conv_w[i - 1], nullptr, c, (long long)C * Lo, Lo, B, C, C,
                            (int)L, (int)Lo, conv_k[i], 1, 0, conv_s[i]);
      cl.out_act = ACT_GELU;
      conv("hub.conv", cl);
      std::swap(a, c);
      L = Lo;
    }
    const long long HL = (long long)H * L;
    float* feats = buf("feats", (size_t)B * C * L);
    launch_copy(feats, a, (long long)B * C * L, s);
    // ---- feature projection: channel LN, 1x1 conv + bias
    float* lnf = buf("feats_ln", (size_t)B * C * L);
    run("hub.ln", 8.0 * B * C * L, 8.0 * B * C * L,
        [&] { launch_layernorm_cols(feats, fp_ln_g, fp_ln_b, lnf, B, C, (int)L, 1e-5f, s); });
    float* proj = buf("proj", (size_t)B * HL);
    conv("hub.proj", c1x1(lnf, (long long)C * L, fp_w, fp_b, proj, B, C, H, (int)L));
    // ---- positional conv in tap blocks (padding pos_k/2, the right column dropped)
    float* pos = buf("pos", (size_t)B * HL);
    if (pos_wl) {
      run("hub.pos", 2.0 * B * (double)H * cpg * pos_k * L,
          4.0 * (2.0 * B * HL + (double)pos_groups * pos_k * cpg * cpg),
          [&] { launch_posconv(proj, pos_wl, pos_b, pos, B, H, (int)L, cpg, pos_k, pos_k / 2, s); });
    }
    for (size_t j = 0; j < pos_w.size(); ++j) {
      const int kb = pos_kb[j];
      ConvLaunch pl{};
      pl.n_groups = pos_groups;
      pl.xb = HL; pl.xc = L; pl.ob = HL; pl.oc = L;
      pl.C_in = cpg; pl.C_out = cpg; pl.w_ld = packed_ld(cpg); pl.L_in = (int)L; pl.B = B; pl.div = 1.f;
      for (int gi = 0; gi < pos_groups; ++gi) {
        ConvGroup& g = pl.g[gi];
        g.x = proj + (long long)gi * cpg * L;
        g.w = pos_w[j] + (size_t)gi * kb * cpg * pl.w_ld;
        g.bias = j == 0 ? pos_b + gi * cpg : nullptr;
        g.res = nullptr;
        g.out = pos + (long long)gi * cpg * L;
        g.K = kb; g.dil = 1; g.in_off = pos_k0[j] - pos_k / 2; g.in_step = 1;
        g.out_step = 1; g.out_off = 0; g.n_out = (int)L;
        g.combine = j == 0 ? COMB_STORE : COMB_ADD;
      }
      conv("hub.pos", pl);
    }
    float* h0 = buf("pos_sum", (size_t)B * HL);
    run("hub.pos", 0.0, 12.0 * B * HL, [&] { launch_add_gelu(h0, proj, pos, (long long)B * HL, s); });
    float* x0 = buf("entry", (size_t)B * HL);
    run("hub.ln", 8.0 * B * HL, 8.0 * B * HL,
        [&] { launch_layernorm_cols(h0, enc_ln_g, enc_ln_b, x0, B, H, (int)L, 1e-5f, s); });
    // ---- transformer layers
    float* qkv = buf("qkv", (size_t)B * 3 * HL);
    float* att = buf("att", (size_t)B * HL);
    float* t1 = buf("t1", (size_t)B * HL);
    float* x1 = buf("x1", (size_t)B * HL);
    float* ff = buf("ffn", (size_t)B * F * L);
    float* xa = buf("xa", (size_t)B * HL);
    float* xb_ = buf("xb", (size_t)B * HL);
    const size_t part_n = std::max<size_t>(1, relpos_attention_scratch_floats(B, kHeads, D, (int)L, 0, false));
    float* part = buf("attn_part", part_n);
    const int nl = version == 1 ? 9 : n_layers;
    // Post-LN layers: x1 = LN1(x + o-proj(attn)), x' = LN2(x1 + FFN(x1)).
    // When the four 1x1 GEMMs of a layer run on the chunked small-conv
    // kernel (L up to about 950 frames), neither LayerNorm is a launch of its
    // own and no normalised tensor is stored: the o-projection and the FFN
    // output GEMM also write the column statistics of their 32-row tiles
    // (st1, st2), the FFN input / next q/k/v GEMM normalise their input while
    // staging it, and the GEMM that adds the normalised tensor as its
    // residual normalises the raw one in its epilogue.  Only the last
    // layer's LN2 is a LayerNorm launch.  Longer inputs (split-K GEMMs) keep
    // the LayerNorm launches.
    const int nt = H / 32;
    double* st1 = reinterpret_cast<double*>(buf("ln_stat1", (size_t)4 * B * nt * L));
    double* st2 = reinterpret_cast<double*>(buf("ln_stat2", (size_t)4 * B * nt * L));
    float* t2 = buf("t2", (size_t)B * HL);
    bool fold = H % 32 == 0;
    {
      const ConvLaunch probe[4] = {c1x1(x0, HL, layers[0].wqkv, layers[0].bqkv, qkv, B, H, 3 * H, (int)L),
                                   c1x1(att, HL, layers[0].wo, layers[0].bo, t1, B, H, H, (int)L),
                                   c1x1(t1, HL, layers[0].wi, layers[0].bi, ff, B, H, F, (int)L),
                                   c1x1(ff, (long long)F * L, layers[0].wf, layers[0].bf, t2, B, F, H, (int)L)};
      for (const ConvLaunch& p : probe) fold = fold && conv1d_mfma_chunked_1x1(p);
    }
    auto ln_in = [&](ConvLaunch& c, const double* st) {  // the affine is in the folded weights
      c.ln_stat = st;
      c.ln_ntile = nt;
      c.ln_eps = 1e-5f;
    };
    auto ln_res = [&](ConvLaunch& c, const double* st, const float* g, const float* bt) {
      c.res_stat = st;
      c.res_g = g;
      c.res_b = bt;
      c.ln_eps = 1e-5f;
    };
    const float* cur = x0;       // the layer input, normalised
    const float* raw = nullptr;  // fold: the previous layer's FFN sum before its LN2 (statistics in st2)
    for (int i = 0; i < nl; ++i) {
      const Layer& Ly = layers[i];
      const Layer* Lp = i > 0 ? &layers[i - 1] : nullptr;
      float* xo = (i & 1) ? xb_ : xa;
      ConvLaunch cq = raw ? c1x1(raw, HL, Ly.wqkv_ln, Ly.bqkv_ln, qkv, B, H, 3 * H, (int)L)
                          : c1x1(cur, HL, Ly.wqkv, Ly.bqkv, qkv, B, H, 3 * H, (int)L);
      if (raw) ln_in(cq, st2);
      conv("hub.qkv", cq);
      run("hub.attn", 4.0 * B * kHeads * (double)L * L * D, 4.0 * B * 4.0 * HL,
          [&] { launch_relpos_attention(qkv, nullptr, nullptr, att, part, part_n, B, kHeads, D, (int)L, 0, s); });
      ConvLaunch co = c1x1(att, HL, Ly.wo, Ly.bo, t1, B, H, H, (int)L);
      co.g[0].res = raw ? raw : cur; co.rb = HL; co.rc = L;
      if (raw) ln_res(co, st2, Lp->ln2_g, Lp->ln2_b);
      if (fold) co.stat_out = st1;
      conv("hub.o", co);
      ConvLaunch fi{};
      if (fold) {
        fi = c1x1(t1, HL, Ly.wi_ln, Ly.bi_ln, ff, B, H, F, (int)L);
        ln_in(fi, st1);
      } else {
        run("hub.ln", 8.0 * B * HL, 8.0 * B * HL,
            [&] { launch_layernorm_cols(t1, Ly.ln1_g, Ly.ln1_b, x1, B, H, (int)L, 1e-5f, s); });
        fi = c1x1(x1, HL, Ly.wi, Ly.bi, ff, B, H, F, (int)L);
      }
      fi.out_act = ACT_GELU;
      conv("hub.ffn", fi);
      float* sum = fold ? t2 : t1;
      ConvLaunch fo = c1x1(ff, (long long)F * L, Ly.wf, Ly.bf, sum, B, F, H, (int)L);
      fo.g[0].res = fold ? t1 : x1; fo.rb = HL; fo.rc = L;
      if (fold) ln_res(fo, st1, Ly.ln1_g, Ly.ln1_b);
      const bool next_folds = fold && i + 1 < nl;
      if (next_folds) fo.stat_out = st2;
      conv("hub.ffn", fo);
      if (next_folds) {
        raw = t2;
        // debug: the layer's output, normalised by a LayerNorm launch (the
        // pipeline itself never stores it)
        if (keep && i == 0)
          launch_layernorm_cols(t2, Ly.ln2_g, Ly.ln2_b, buf("layer1", (size_t)B * HL), B, H, (int)L, 1e-5f, s);
      } else {
        run("hub.ln", 8.0 * B * HL, 8.0 * B * HL,
            [&] { launch_layernorm_cols(sum, Ly.ln2_g, Ly.ln2_b, xo, B, H, (int)L, 1e-5f, s); });
        cur = xo;
        raw = nullptr;
        if (keep && i == 0) launch_copy(buf("layer1", (size_t)B * HL), xo, (long long)B * HL, s);
      }
    }
    const int od = out_dim(version);
    const float* res = cur;
    if (version == 1) {
      float* fpj = buf("final", (size_t)B * od * L);
      conv("hub.final", c1x1(cur, HL, final_w, final_b, fpj, B, H, od, (int)L));
      res = fpj;
    }
    launch_transpose(res, out, B, od, (int)L, 1.0f, s);
  }
};

namespace {
std::mutex g_hub_mu;
std::unordered_map<long long, Hubert*> g_hubs;
long long g_next_hub = 1;

Hubert* hub_from(long long h) {
  std::lock_guard<std::mutex> lk(g_hub_mu);
  auto it = g_hubs.find(h);
  return it == g_hubs.end() ? nullptr : it->second;
}
}  // namespace

}  // namespace rvc

using namespace rvc;

template <class F>
static int32_t hguard(int64_t hh, F&& body) {
  Hubert* s = hub_from(hh);
  if (!s) {
    set_last_error("invalid hubert handle");
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

int64_t rvc_hubert_create(int64_t h) {
  Engine* e = engine_from_handle(h);
  if (!e) {
    set_last_error("invalid engine handle");
    return -1;
  }
  Hubert* s = new Hubert();
  s->eng = e;
  std::lock_guard<std::mutex> lk(g_hub_mu);
  const long long id = g_next_hub++;
  g_hubs[id] = s;
  return id;
}

int32_t rvc_hubert_destroy(int64_t hh) {
  Hubert* s = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_hub_mu);
    auto it = g_hubs.find(hh);
    if (it == g_hubs.end()) {
      set_last_error("invalid hubert handle");
      return -1;
    }
    s = it->second;
    g_hubs.erase(it);
  }
  {
    std::lock_guard<std::mutex> lk(s->eng->mu);
    delete s;
  }
  return 0;
}

int32_t rvc_hubert_set_weight(int64_t hh, const char* key, const float* data, const int64_t* shape, int32_t ndim) {
  return hguard(hh, [&](Hubert& s) { s.set_weight(key, data, shape, ndim); });
}

int32_t rvc_hubert_finalize(int64_t hh) {
  return hguard(hh, [&](Hubert& s) { s.finalize(); });
}

int32_t rvc_hubert_frames(int64_t hh, int64_t T, int64_t* L) {
  return hguard(hh, [&](Hubert& s) {
    RVC_CHECK(s.ready && L && T >= 0, "frames: invalid arguments");
    *L = s.frames(T);
  });
}

int32_t rvc_hubert_encode(int64_t hh, const float* x, int64_t B, int64_t T, int32_t version, float* out) {
  return hguard(hh, [&](Hubert& s) {
    s.check_args(B, T, version);
    RVC_CHECK(x && out, "encode: null pointer");
    hipStream_t st = s.eng->stream;
    const long long L = s.frames(T);
    const long long n_out = (long long)B * L * s.out_dim(version);
    float* dx = s.buf("in_x", (size_t)(B * T));
    float* dout = s.buf("out", (size_t)n_out);
    RVC_HIP(hipMemcpyAsync(dx, x, sizeof(float) * B * T, hipMemcpyHostToDevice, st));
    s.encode(dx, (int)B, T, version, dout);
    s.close_span();
    RVC_HIP(hipMemcpyAsync(out, dout, sizeof(float) * n_out, hipMemcpyDeviceToHost, st));
    RVC_HIP(hipStreamSynchronize(st));
    s.collect_timing();
  });
}

int32_t rvc_hubert_encode_dev(int64_t hh, int64_t x, int64_t B, int64_t T, int32_t version, int64_t out) {
  return hguard(hh, [&](Hubert& s) {
    s.check_args(B, T, version);
    Engine& e = *s.eng;
    const long long L = s.frames(T);
    const float* xp = e.fptr(x, B * T, "hubert x");
    float* op = e.fptr(out, B * L * s.out_dim(version), "hubert out");
    s.encode(xp, (int)B, T, version, op);
    s.close_span();
    e.sync();
    s.collect_timing();
  });
}

int32_t rvc_hubert_read(int64_t hh, const char* name, float* dst, int64_t n) {
  return hguard(hh, [&](Hubert& s) {
    RVC_CHECK(name && dst && n >= 0, "read: invalid arguments");
    s.read(name, dst, n);
  });
}

int32_t rvc_hubert_set_debug(int64_t hh, int32_t keep) {
  return hguard(hh, [&](Hubert& s) { s.keep = keep != 0; });
}

int32_t rvc_hubert_set_timing(int64_t hh, const char* tag) {
  return hguard(hh, [&](Hubert& s) { s.set_timing(tag); });
}

int32_t rvc_hubert_get_timing(int64_t hh, double* total_ms, int64_t* launches, double* flops, double* bytes) {
  return hguard(hh, [&](Hubert& s) {
    if (total_ms) *total_ms = s.t_ms;
    if (launches) *launches = s.t_n;
    if (flops) *flops = s.t_flops;
    if (bytes) *bytes = s.t_bytes;
  });
}

}  // extern "C"
