// Device-resident RMVPE pitch extractor session (rvc_rmvpe_* exports).
//
// Runs RMVPE.infer_from_audio (runtime/models/rmvpe.py:927-952) on one stream:
//   mel front end  :632-640  reflect-padded hop blocks -> windowed DFT as a
//                            7-tap conv1d GEMM (1026 Re/Im rows) -> |X| ->
//                            HTK mel GEMM -> log(clamp 1e-5) -> frames padded
//                            to a multiple of 32 and the input BatchNorm,
//                            written as the [F', 128] image (:861-868)
//   U-Net          :643-690  5 encoder levels of 4 ConvBlockRes (BN folded
//                            into the conv weights, ReLU and the residual in
//                            the epilogue; the 1x1 shortcut first, the second
//                            conv adds onto it) each followed by 2x2 average
//                            pooling; 4 intermediate levels; 5 decoder levels:
//                            ConvTranspose2d as four polyphase groups written
//                            straight into the first half of the level's
//                            concat buffer, whose second half the encoder
//                            level wrote, then 4 ConvBlockRes
//   head           :735-751  cnn 3x3 conv written as [3*128][F'] (the
//                            transpose/reshape for the GRU), GRU input GEMM
//                            for both directions, the BiGRU recurrence, the
//                            Linear(512, 360) GEMM with the sigmoid fused
//   decode         :899-924  argmax + local-average cents, threshold, Hz
// Everything is float32; the numbers follow the reference within rounding.
#include <cmath>
#include <cstring>

#include "../../include/rvc_hip.h"
#include "session.h"

namespace rvc {

struct Rmvpe : SessionBase {
  static constexpr int kHop = 160, kNfft = 1024, kBins = kNfft / 2 + 1, kMels = 128, kTaps = 7;
  static constexpr int kLevels = 5, kInter = 4, kBlocks = 4;
  static constexpr long long kGruSpin = 1LL << 22;

  struct Block {
    int ci = 0, co = 0;
    float *w0 = nullptr, *b0 = nullptr, *w3 = nullptr, *b3 = nullptr, *ws = nullptr, *bs = nullptr;
  };
  struct Up {
    int ci = 0, co = 0;
    float* w[4] = {nullptr, nullptr, nullptr, nullptr};
    float* b = nullptr;
  };
  std::vector<Block> blocks;  // encoder, intermediate, decoder order
  std::vector<Up> ups;
  std::vector<int> en;        // encoder level widths
  int inter = 0, gru_h = 0, gru_in = 0, nbins = 0;
  float bn_s = 1.f, bn_t = 0.f;
  float *cnn_w = nullptr, *cnn_b = nullptr;
  int cnn_co = 0;
  float *wih = nullptr, *bih = nullptr, *whh = nullptr, *bhh = nullptr;
  float *fc_w = nullptr, *fc_b = nullptr;
  float *dft_w = nullptr, *mel_w = nullptr, *cents = nullptr;

  // ---------------------------------------------------------------- weights
  std::pair<std::vector<float>, std::vector<float>> bn(const std::string& p) const {
    const HostT& g = W(p + ".weight");
    const HostT& b = W(p + ".bias");
    const HostT& rm = W(p + ".running_mean");
    const HostT& rv = W(p + ".running_var");
    const size_t n = g.data.size();
    RVC_CHECK(b.data.size() == n && rm.data.size() == n && rv.data.size() == n, p + ": BatchNorm sizes differ");
    std::vector<float> s(n), t(n);
    for (size_t i = 0; i < n; ++i) {
      s[i] = g.data[i] / std::sqrt(rv.data[i] + 1e-5f);   // rmvpe.py:507-515, float32
      t[i] = b.data[i] - rm.data[i] * s[i];
    }
    return {s, t};
  }

  float* conv_folded(const std::string& key, const std::string& bnp, int co, int ci, float** bias) {
    const HostT& w = W(key);
    check_shape(key, w.shape, {co, ci, 3, 3});
    auto st = bn(bnp);
    RVC_CHECK((int)st.first.size() == co, bnp + ": expected one entry per output channel");
    *bias = upload(st.second);
    return upload(pack_conv2d_host(w.data.data(), st.first.data(), co, ci, 3, 3));
  }

  Block make_block(const std::string& p, int ci, int co) {
    Block b;
    b.ci = ci;
    b.co = co;
    b.w0 = conv_folded(p + ".conv.0.weight", p + ".conv.1", co, ci, &b.b0);
    b.w3 = conv_folded(p + ".conv.3.weight", p + ".conv.4", co, co, &b.b3);
    if (has(p + ".shortcut.weight")) {
      const HostT& w = W(p + ".shortcut.weight");
      check_shape(p + ".shortcut.weight", w.shape, {co, ci, 1, 1});
      b.ws = upload(pack_conv2d_host(w.data.data(), nullptr, co, ci, 1, 1));
      b.bs = has(p + ".shortcut.bias") ? upload_vec(p + ".shortcut.bias", co) : nullptr;
    } else {
      RVC_CHECK(ci == co, p + ": channel change without a shortcut conv");
    }
    return b;
  }

  // ConvTranspose2d 3x3 s2 p1 op1 phases: output row 2a + ph reads input row
  // a + dh with kernel row kh: ph 0 -> (dh 0, kh 1); ph 1 -> (dh 1, kh 0),
  // (dh 0, kh 2).  Columns alike.
  static void phase_taps(int ph, int pw, std::vector<int>& dh, std::vector<int>& dw, std::vector<int>& kh,
                         std::vector<int>& kw) {
    std::vector<std::pair<int, int>> rt = ph == 0 ? std::vector<std::pair<int, int>>{{0, 1}}
                                                  : std::vector<std::pair<int, int>>{{1, 0}, {0, 2}};
    std::vector<std::pair<int, int>> ct = pw == 0 ? std::vector<std::pair<int, int>>{{0, 1}}
                                                  : std::vector<std::pair<int, int>>{{1, 0}, {0, 2}};
    dh.clear(); dw.clear(); kh.clear(); kw.clear();
    for (auto& r : rt)
      for (auto& c : ct) {
        dh.push_back(r.first); kh.push_back(r.second);
        dw.push_back(c.first); kw.push_back(c.second);
      }
  }

  Up make_up(const std::string& p, int ci, int co) {
    Up u;
    u.ci = ci;
    u.co = co;
    const HostT& w = W(p + ".conv1.0.weight");
    check_shape(p + ".conv1.0.weight", w.shape, {ci, co, 3, 3});
    auto st = bn(p + ".conv1.1");
    RVC_CHECK((int)st.first.size() == co, p + ".conv1.1: expected one entry per output channel");
    u.b = upload(st.second);
    const int ld = packed_ld(co);
    for (int ph = 0; ph < 2; ++ph)
      for (int pw = 0; pw < 2; ++pw) {
        std::vector<int> dh, dw, kh, kw;
        phase_taps(ph, pw, dh, dw, kh, kw);
        std::vector<float> pk((size_t)dh.size() * ci * ld, 0.f);
        for (size_t t = 0; t < dh.size(); ++t)
          for (int c = 0; c < ci; ++c)
            for (int o = 0; o < co; ++o)
              pk[(t * ci + c) * ld + o] = w.data[(((size_t)c * co + o) * 3 + kh[t]) * 3 + kw[t]] * st.first[o];
        u.w[ph * 2 + pw] = upload(pk);
      }
    return u;
  }

  // windowed DFT as conv1d weights [7][160][ld(1026)]: tap k, channel c is
  // frame sample n = 160 k + c; rows 0..512 Re (cos), 513..1025 Im (-sin)
  std::vector<float> dft_pack() const {
    const int Co = 2 * kBins, ld = packed_ld(Co);
    std::vector<float> o((size_t)kTaps * kHop * ld, 0.f);
    for (int k = 0; k < kTaps; ++k)
      for (int c = 0; c < kHop; ++c) {
        const int n = k * kHop + c;
        if (n >= kNfft) continue;
        const double win = 0.5 - 0.5 * std::cos(2.0 * M_PI * n / (kNfft - 1));   // np.hanning
        for (int b = 0; b < kBins; ++b) {
          const double ang = 2.0 * M_PI * (double)(((long long)b * n) % kNfft) / kNfft;
          o[((size_t)k * kHop + c) * ld + b] = (float)(win * std::cos(ang));
          o[((size_t)k * kHop + c) * ld + kBins + b] = (float)(-win * std::sin(ang));
        }
      }
    return o;
  }

  // HTK mel filters with unit row sums (runtime/dsp/mel.py:68-122), packed
  // as 1x1 conv weights [1][513][128]
  static std::vector<float> mel_pack() {
    const double sr = 16000.0, fmin = 30.0, fmax = 8000.0;
    auto hz2mel = [](double f) { return 1127.0 * std::log1p(f / 700.0); };
    const double m0 = hz2mel(fmin), m1 = hz2mel(fmax);
    std::vector<double> edges(kMels + 2);
    const double step = (m1 - m0) / (kMels + 1);
    for (int i = 0; i < kMels + 2; ++i) {
      const double m = i == kMels + 1 ? m1 : i * step + m0;   // np.linspace (exact end point)
      edges[i] = 700.0 * std::expm1(m / 1127.0);
    }
    const int ld = packed_ld(kMels);
    std::vector<float> o((size_t)kBins * ld, 0.f);
    std::vector<double> tri(kBins);
    for (int i = 0; i < kMels; ++i) {
      const double lo = edges[i], c = edges[i + 1], hi = edges[i + 2];
      double tot = 0;
      for (int b = 0; b < kBins; ++b) {
        const double f = sr / 2.0 * b / (kBins - 1);
        const double up = c > lo ? (f - lo) / (c - lo) : 0.0;
        const double dn = hi > c ? (hi - f) / (hi - c) : 0.0;
        tri[b] = std::max(0.0, std::min(up, dn));
        tot += tri[b];
      }
      for (int b = 0; b < kBins; ++b) o[(size_t)b * ld + i] = (float)(tot > 0 ? tri[b] / tot : tri[b]);
    }
    return o;
  }

  void finalize() {
    RVC_CHECK(!ready, "rmvpe session already finalized");
    // architecture from the checkpoint's shapes (E2E(4, 1, (2, 2)))
    en.clear();
    int c = 1;
    for (int i = 0; i < kLevels; ++i) {
      const std::string p = "unet.encoder.layers." + std::to_string(i) + ".conv.0.conv.0.weight";
      const HostT& w = W(p);
      RVC_CHECK(w.shape.size() == 4 && w.shape[1] == c, p + ": unexpected input channels");
      en.push_back((int)w.shape[0]);
      c = en.back();
    }
    inter = (int)W("unet.intermediate.layers.0.conv.0.conv.0.weight").shape[0];
    auto e_bn = bn("unet.encoder.bn");
    RVC_CHECK(e_bn.first.size() == 1, "unet.encoder.bn must have one channel");
    bn_s = e_bn.first[0];
    bn_t = e_bn.second[0];
    blocks.clear();
    ups.clear();
    c = 1;
    for (int i = 0; i < kLevels; ++i) {
      for (int j = 0; j < kBlocks; ++j)
        blocks.push_back(make_block("unet.encoder.layers." + std::to_string(i) + ".conv." + std::to_string(j),
                                    j == 0 ? c : en[i], en[i]));
      c = en[i];
    }
    for (int i = 0; i < kInter; ++i) {
      for (int j = 0; j < kBlocks; ++j)
        blocks.push_back(make_block("unet.intermediate.layers." + std::to_string(i) + ".conv." + std::to_string(j),
                                    j == 0 ? c : inter, inter));
      c = inter;
    }
    for (int i = 0; i < kLevels; ++i) {
      const int co = en[kLevels - 1 - i];
      const std::string p = "unet.decoder.layers." + std::to_string(i);
      ups.push_back(make_up(p, c, co));
      for (int j = 0; j < kBlocks; ++j)
        blocks.push_back(make_block(p + ".conv2." + std::to_string(j), j == 0 ? 2 * co : co, co));
      c = co;
    }
    const HostT& cw = W("cnn.weight");
    RVC_CHECK(cw.shape.size() == 4 && cw.shape[1] == c && cw.shape[2] == 3 && cw.shape[3] == 3,
              "cnn.weight: expected [C, en0, 3, 3]");
    cnn_co = (int)cw.shape[0];
    cnn_w = upload(pack_conv2d_host(cw.data.data(), nullptr, cnn_co, c, 3, 3));
    cnn_b = upload_vec("cnn.bias", cnn_co);
    const std::string g = "fc.0.gru.";
    const HostT& wi = W(g + "weight_ih_l0");
    RVC_CHECK(wi.shape.size() == 2 && wi.shape[0] % 3 == 0, "GRU weight_ih must be [3H, in]");
    gru_h = (int)wi.shape[0] / 3;
    gru_in = (int)wi.shape[1];
    RVC_CHECK(gru_h >= 1 && gru_h <= 256, "GRU hidden size must be 1..256");
    RVC_CHECK(gru_in == cnn_co * kMels, "GRU input must be cnn channels x 128 mel bins");
    {
      std::vector<float> wcat;
      std::vector<float> bcat, hcat, bhcat;
      for (const char* sfx : {"", "_reverse"}) {
        const HostT& a = W(g + "weight_ih_l0" + sfx);
        check_shape(g + "weight_ih_l0" + sfx, a.shape, {3 * gru_h, gru_in});
        wcat.insert(wcat.end(), a.data.begin(), a.data.end());
        const HostT& b = W(g + "bias_ih_l0" + sfx);
        check_shape(g + "bias_ih_l0" + sfx, b.shape, {3 * gru_h});
        bcat.insert(bcat.end(), b.data.begin(), b.data.end());
        const HostT& h = W(g + "weight_hh_l0" + sfx);
        check_shape(g + "weight_hh_l0" + sfx, h.shape, {3 * gru_h, gru_h});
        hcat.insert(hcat.end(), h.data.begin(), h.data.end());
        const HostT& bh = W(g + "bias_hh_l0" + sfx);
        check_shape(g + "bias_hh_l0" + sfx, bh.shape, {3 * gru_h});
        bhcat.insert(bhcat.end(), bh.data.begin(), bh.data.end());
      }
      wih = upload(pack(wcat, 6 * gru_h, gru_in, 1));
      bih = upload(bcat);
      whh = upload(hcat);
      bhh = upload(bhcat);
    }
    const HostT& fw = W("fc.1.weight");
    RVC_CHECK(fw.shape.size() == 2 && fw.shape[1] == 2 * gru_h, "fc.1.weight must be [bins, 2H]");
    nbins = (int)fw.shape[0];
    fc_w = upload(pack(fw.data, nbins, 2 * gru_h, 1));
    fc_b = upload_vec("fc.1.bias", nbins);
    dft_w = upload(dft_pack());
    mel_w = upload(mel_pack());
    std::vector<float> ct(nbins + 8, 0.f);
    for (int i = 0; i < nbins; ++i) ct[i + 4] = (float)(20.0 * i + 1997.3794084376191);   // rmvpe.py:565-566
    cents = upload(ct);
    host.clear();
    ready = true;
  }

  // ---------------------------------------------------------------- launches
  // "same" conv on a [C][H][W] image: 3x3 (pad 1) or 1x1
  void conv2(const char* t, const float* x, int ci, int H, int Wd, const float* w, int k, const float* bias, bool relu,
             const float* res, float* out, int co) {
    Conv2dLaunch a{};
    a.n_groups = 1;
    Conv2dGroup& g = a.g[0];
    g.w = w;
    g.ntaps = k * k;
    for (int i = 0; i < k; ++i)
      for (int j = 0; j < k; ++j) {
        g.dh[i * k + j] = i - (k - 1) / 2;
        g.dw[i * k + j] = j - (k - 1) / 2;
      }
    g.oh0 = g.ow0 = 0;
    g.a_lim = H;
    g.b_lim = Wd;
    g.oh_n = H;
    g.ow_n = Wd;
    a.x = x; a.xb = (long long)ci * H * Wd; a.xc = (long long)H * Wd; a.H = H; a.W = Wd;
    a.out = out; a.ob = (long long)co * H * Wd; a.oc = (long long)H * Wd; a.ors = Wd; a.ocs = 1;
    a.res = res; a.bias = bias; a.relu = relu ? 1 : 0;
    a.C_in = ci; a.C_out = co; a.w_ld = packed_ld(co); a.B = 1;
    a.OH = H; a.OW = Wd; a.osh = a.osw = 1; a.stride = 1;
    launch2(t, a);
  }
  void launch2(const char* t, Conv2dLaunch a) {
    double taps = 0;
    for (int i = 0; i < a.n_groups; ++i) taps += a.g[i].ntaps;
    const double pts = (double)a.B * a.OH * a.OW;
    const double flops = 2.0 * pts * a.C_in * a.C_out * taps;
    const double bytes = 4.0 * ((double)a.B * a.C_in * a.H * a.W + pts * a.C_out * a.n_groups * (a.res ? 2 : 1));
    const size_t need = conv2d_split_floats(a);
    if (need > 0) {
      a.part = buf("c2split", need);
      a.part_floats = need;
    }
    run(t, flops, bytes, [&] { launch_conv2d(a, eng->stream); });
  }

  void block(const char* t, const Block& b, const float* x, int H, int Wd, float* tmp, float* dst) {
    conv2(t, x, b.ci, H, Wd, b.w0, 3, b.b0, true, nullptr, tmp, b.co);
    const float* res = x;
    if (b.ws) {
      conv2(t, x, b.ci, H, Wd, b.ws, 1, b.bs, false, nullptr, dst, b.co);
      res = dst;
    }
    conv2(t, tmp, b.co, H, Wd, b.w3, 3, b.b3, true, res, dst, b.co);
  }

  // ConvTranspose2d (+ folded BN + ReLU) of x [ci][H][W] into out [co][2H][2W]
  void up(const char* t, const Up& u, const float* x, int H, int Wd, float* out) {
    Conv2dLaunch a{};
    a.n_groups = 4;
    for (int ph = 0; ph < 2; ++ph)
      for (int pw = 0; pw < 2; ++pw) {
        Conv2dGroup& g = a.g[ph * 2 + pw];
        std::vector<int> dh, dw, kh, kw;
        phase_taps(ph, pw, dh, dw, kh, kw);
        g.w = u.w[ph * 2 + pw];
        g.ntaps = (int)dh.size();
        for (int i = 0; i < g.ntaps; ++i) {
          g.dh[i] = dh[i];
          g.dw[i] = dw[i];
        }
        g.oh0 = ph;
        g.ow0 = pw;
        // the reference leaves output row 2H-1 / column 2W-1 without taps
        // (symmetric padding + zero-filled output padding, rmvpe.py:369-383)
        g.a_lim = ph ? H - 1 : H;
        g.b_lim = pw ? Wd - 1 : Wd;
        g.oh_n = H;
        g.ow_n = Wd;
      }
    a.x = x; a.xb = (long long)u.ci * H * Wd; a.xc = (long long)H * Wd; a.H = H; a.W = Wd;
    a.out = out; a.ob = (long long)u.co * 4 * H * Wd; a.oc = 4LL * H * Wd; a.ors = 2 * Wd; a.ocs = 1;
    a.res = nullptr; a.bias = u.b; a.relu = 1;
    a.C_in = u.ci; a.C_out = u.co; a.w_ld = packed_ld(u.co); a.B = 1;
    a.OH = H; a.OW = Wd; a.osh = a.osw = 2; a.stride = 1;
    launch2(t, a);
  }

  static int frames(long long T) { return (int)(1 + T / kHop); }
  static int padded(int F) { return 32 * ((F - 1) / 32 + 1); }

  size_t image_cap(int Fp) const {
    size_t cap = 0;
    int H = Fp, Wd = kMels;
    for (int i = 0; i < kLevels; ++i) {
      cap = std::max(cap, (size_t)en[i] * H * Wd);
      H /= 2;
      Wd /= 2;
    }
    cap = std::max(cap, (size_t)inter * H * Wd);
    return cap;
  }

  // audio x [T] (device) -> f0 [F] (device)
  void infer(const float* x, long long T, float thred, float* f0) {
    hipStream_t s = eng->stream;
    const int F = frames(T), Fp = padded(F), NB = F + kTaps - 1;
    // ---- mel front end
    float* xb = buf("blocks", (size_t)kHop * NB);
    run("rmvpe.mel", 0.0, 4.0 * kHop * NB * 2, [&] { launch_rmvpe_blocks(x, (int)T, xb, NB, s); });
    float* S = buf("stft", (size_t)2 * kBins * F);
    {
      ConvLaunch a = cargs(xb, (long long)kHop * NB, NB, dft_w, nullptr, S, (long long)2 * kBins * F, F, 1, kHop,
                           2 * kBins, NB, F, kTaps, 1, 0);
      conv("rmvpe.mel", a);
    }
    float* mag = buf("mag", (size_t)kBins * F);
    run("rmvpe.mel", 0.0, 12.0 * kBins * F, [&] { launch_mel_mag(S, mag, kBins, F, s); });
    float* M = buf("melpow", (size_t)kMels * F);
    conv("rmvpe.mel", c1x1(mag, (long long)kBins * F, mel_w, nullptr, M, 1, kBins, kMels, F));
    float* img = buf("image", (size_t)Fp * kMels);
    float* lm = buf("mel", (size_t)kMels * F);
    run("rmvpe.mel", 0.0, 4.0 * (kMels * F * 2.0 + Fp * kMels),
        [&] { launch_logmel_image(M, F, Fp, kMels, bn_s, bn_t, img, lm, s); });
    // ---- U-Net
    const size_t cap = image_cap(Fp);
    float* pp[2] = {buf("pp0", cap), buf("pp1", cap)};
    float* tmp = buf("tmp", cap);
    std::vector<float*> cat(kLevels);
    int H = Fp, Wd = kMels, c = 1;
    const float* cur = img;
    size_t bi = 0;
    for (int i = 0; i < kLevels; ++i) {
      cat[i] = buf("cat" + std::to_string(i), (size_t)2 * en[i] * H * Wd);
      for (int j = 0; j < kBlocks; ++j, ++bi) {
        float* dst = j == kBlocks - 1 ? cat[i] + (size_t)en[i] * H * Wd : (cur == pp[0] ? pp[1] : pp[0]);
        block("rmvpe.enc", blocks[bi], cur, H, Wd, tmp, dst);
        cur = dst;
      }
      c = en[i];
      run("rmvpe.pool", 0.0, 5.0 * c * H * Wd, [&] { launch_avg_pool2(cur, pp[0], c, H, Wd, s); });
      cur = pp[0];
      H /= 2;
      Wd /= 2;
    }
    for (int i = 0; i < kInter; ++i)
      for (int j = 0; j < kBlocks; ++j, ++bi) {
        float* dst = cur == pp[0] ? pp[1] : pp[0];
        block("rmvpe.inter", blocks[bi], cur, H, Wd, tmp, dst);
        cur = dst;
      }
    for (int i = 0; i < kLevels; ++i) {
      const int k = kLevels - 1 - i;
      up("rmvpe.dec", ups[i], cur, H, Wd, cat[k]);
      H *= 2;
      Wd *= 2;
      cur = cat[k];
      for (int j = 0; j < kBlocks; ++j, ++bi) {
        float* dst = cur == pp[0] ? pp[1] : pp[0];
        block("rmvpe.dec", blocks[bi], cur, H, Wd, tmp, dst);
        cur = dst;
      }
    }
    // ---- head
    const int Cx = cnn_co * kMels;
    float* X = buf("gru_in", (size_t)Cx * Fp);
    {
      Conv2dLaunch a{};
      a.n_groups = 1;
      Conv2dGroup& g = a.g[0];
      g.w = cnn_w;
      g.ntaps = 9;
      for (int t = 0; t < 9; ++t) {
        g.dh[t] = t / 3 - 1;
        g.dw[t] = t % 3 - 1;
      }
      g.a_lim = Fp;
      g.b_lim = kMels;
      g.oh_n = Fp;
      g.ow_n = kMels;
      a.x = cur; a.xb = (long long)en[0] * Fp * kMels; a.xc = (long long)Fp * kMels; a.H = Fp; a.W = kMels;
      // (c, h, w) -> row c*128 + w, column h: the reference's
      // transpose(0, 2, 1, 3).reshape(F', 384), channel-major for the GEMM
      a.out = X; a.ob = (long long)Cx * Fp; a.oc = (long long)kMels * Fp; a.ors = 1; a.ocs = Fp;
      a.bias = cnn_b;
      a.C_in = en[0]; a.C_out = cnn_co; a.w_ld = packed_ld(cnn_co); a.B = 1;
      a.OH = Fp; a.OW = kMels; a.osh = a.osw = 1; a.stride = 1;
      launch2("rmvpe.head", a);
    }
    float* GX = buf("gru_gx", (size_t)6 * gru_h * Fp);
    conv("rmvpe.head", c1x1(X, (long long)Cx * Fp, wih, bih, GX, 1, Cx, 6 * gru_h, Fp));
    float* HO = buf("gru_out", (size_t)2 * gru_h * Fp);
    auto* state = reinterpret_cast<unsigned long long*>(buf("gru_state", 2 * 2 * 256 * 2));
    unsigned* sync = reinterpret_cast<unsigned*>(buf("gru_sync", 4));
    {
      GruArgs ga{};
      ga.gx = GX; ga.g_d = (long long)3 * gru_h * Fp; ga.g_t = 1; ga.g_r = Fp;
      ga.whh = whh; ga.bhh = bhh;
      ga.out = HO; ga.o_d = (long long)gru_h * Fp; ga.o_t = 1; ga.o_j = Fp;
      ga.state = state; ga.sync = sync;
      ga.T = Fp; ga.H = gru_h; ga.spin_limit = kGruSpin;
      run("rmvpe.gru", 2.0 * 2 * Fp * 3.0 * gru_h * gru_h, 4.0 * 2 * Fp * 4.0 * gru_h,
          [&] { launch_bigru(ga, s); });
    }
    float* SAL = buf("salience", (size_t)nbins * Fp);
    {
      ConvLaunch a = c1x1(HO, (long long)2 * gru_h * Fp, fc_w, fc_b, SAL, 1, 2 * gru_h, nbins, Fp);
      a.out_act = ACT_SIGMOID;
      conv("rmvpe.head", a);
    }
    run("rmvpe.decode", 0.0, 4.0 * nbins * F,
        [&] { launch_rmvpe_decode(SAL, 1, Fp, F, nbins, cents, thred, f0, s); });
  }

  void check_gru() {
    unsigned flag = 0;
    auto it = ws.find("gru_sync");
    if (it == ws.end()) return;
    RVC_HIP(hipMemcpyAsync(&flag, reinterpret_cast<unsigned*>(it->second.first) + 2, sizeof(unsigned),
                           hipMemcpyDeviceToHost, eng->stream));
    RVC_HIP(hipStreamSynchronize(eng->stream));
    RVC_CHECK(flag == 0, "rmvpe: BiGRU step barrier timed out (workgroups not co-resident)");
  }

  void check_T(long long T) const {
    RVC_CHECK(ready, "rmvpe session not finalized");
    RVC_CHECK(T > kNfft / 2 && T <= (1LL << 28), "rmvpe: audio must hold more than 512 samples");
  }
};

namespace {
std::mutex g_rmvpe_mu;
std::unordered_map<long long, Rmvpe*> g_rmvpes;
long long g_next_rmvpe = 1;

Rmvpe* rmvpe_from(long long h) {
  std::lock_guard<std::mutex> lk(g_rmvpe_mu);
  auto it = g_rmvpes.find(h);
  return it == g_rmvpes.end() ? nullptr : it->second;
}
}  // namespace

}  // namespace rvc

using namespace rvc;

template <class F>
static int32_t rguard(int64_t hh, F&& body) {
  Rmvpe* s = rmvpe_from(hh);
  if (!s) {
    set_last_error("invalid rmvpe handle");
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

int64_t rvc_rmvpe_create(int64_t h) {
  Engine* e = engine_from_handle(h);
  if (!e) {
    set_last_error("invalid engine handle");
    return -1;
  }
  Rmvpe* s = new Rmvpe();
  s->eng = e;
  std::lock_guard<std::mutex> lk(g_rmvpe_mu);
  const long long id = g_next_rmvpe++;
  g_rmvpes[id] = s;
  return id;
}

int32_t rvc_rmvpe_destroy(int64_t hh) {
  Rmvpe* s = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_rmvpe_mu);
    auto it = g_rmvpes.find(hh);
    if (it == g_rmvpes.end()) {
      set_last_error("invalid rmvpe handle");
      return -1;
    }
    s = it->second;
    g_rmvpes.erase(it);
  }
  {
    std::lock_guard<std::mutex> lk(s->eng->mu);
    delete s;
  }
  return 0;
}

int32_t rvc_rmvpe_set_weight(int64_t hh, const char* key, const float* data, const int64_t* shape, int32_t ndim) {
  return rguard(hh, [&](Rmvpe& s) { s.set_weight(key, data, shape, ndim); });
}

int32_t rvc_rmvpe_finalize(int64_t hh) {
  return rguard(hh, [&](Rmvpe& s) { s.finalize(); });
}

int32_t rvc_rmvpe_frames(int64_t hh, int64_t T, int64_t* F) {
  return rguard(hh, [&](Rmvpe& s) {
    RVC_CHECK(F && T >= 0, "frames: invalid arguments");
    *F = Rmvpe::frames(T);
  });
}

int32_t rvc_rmvpe_infer(int64_t hh, const float* x, int64_t T, double thred, float* f0) {
  return rguard(hh, [&](Rmvpe& s) {
    s.check_T(T);
    RVC_CHECK(x && f0, "infer: null pointer");
    hipStream_t st = s.eng->stream;
    const int F = Rmvpe::frames(T);
    float* dx = s.buf("in_x", (size_t)T);
    float* df = s.buf("out_f0", (size_t)F);
    RVC_HIP(hipMemcpyAsync(dx, x, sizeof(float) * T, hipMemcpyHostToDevice, st));
    s.infer(dx, T, (float)thred, df);
    s.close_span();
    RVC_HIP(hipMemcpyAsync(f0, df, sizeof(float) * F, hipMemcpyDeviceToHost, st));
    RVC_HIP(hipStreamSynchronize(st));
    s.check_gru();
    s.collect_timing();
  });
}

int32_t rvc_rmvpe_infer_dev(int64_t hh, int64_t x, int64_t T, double thred, int64_t f0) {
  return rguard(hh, [&](Rmvpe& s) {
    s.check_T(T);
    Engine& e = *s.eng;
    const float* xp = e.fptr(x, T, "rmvpe audio");
    float* fp = e.fptr(f0, Rmvpe::frames(T), "rmvpe f0");
    s.infer(xp, T, (float)thred, fp);
    s.close_span();
    e.sync();
    s.check_gru();
    s.collect_timing();
  });
}

int32_t rvc_rmvpe_read(int64_t hh, const char* name, float* dst, int64_t n) {
  return rguard(hh, [&](Rmvpe& s) {
    RVC_CHECK(name && dst && n >= 0, "read: invalid arguments");
    s.read(name, dst, n);
  });
}

int32_t rvc_rmvpe_set_timing(int64_t hh, const char* tag) {
  return rguard(hh, [&](Rmvpe& s) { s.set_timing(tag); });
}

int32_t rvc_rmvpe_get_timing(int64_t hh, double* total_ms, int64_t* launches, double* flops, double* bytes) {
  return rguard(hh, [&](Rmvpe& s) {
    if (total_ms) *total_ms = s.t_ms;
    if (launches) *launches = s.t_n;
    if (flops) *flops = s.t_flops;
    if (bytes) *bytes = s.t_bytes;
  });
}

}  // extern "C"
