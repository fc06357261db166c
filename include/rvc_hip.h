/*
 * rvc_hip.h -- C ABI of the MI355X (gfx950) HIP backend for RVC's synthesis
 * hot path (GeneratorNSF + enc_p + flow).
 *
 * The library (librvc_hip.so) is a drop-in for the reference's native engine
 * at its C boundary: same export names, argument order and meaning, and the
 * same conventions (engine/src/ffi.zig:1-45):
 *   - every export returns int32 0 on success, -1 on failure; the message is
 *     kept in a process-global, mutex-protected buffer read with
 *     rvc_last_error;
 *   - rvc_engine_create returns an int64 handle (> 0) or -1;
 *   - buffer ids are opaque int64 keys; id 0 means "no bias";
 *   - sizes are float counts, except rvc_mem_alloc / rvc_mem_fill_zero /
 *     *_bytes which take bytes;
 *   - f32 scalars (leaky slope, batch layer-norm eps, transpose scale) travel
 *     as IEEE-754 bit patterns in the low 32 bits of an int64
 *     (runtime/vulkan_ops.py:255-261);
 *   - every call on one engine is serialised by that engine's mutex.
 * Differences from the reference engine: handles are table keys, not raw
 * pointers (a stale handle is rejected); single ops are enqueued on the
 * engine's HIP stream and complete before any download returns.
 *
 * Everything below the ABI is new MI355X code: fp32 MFMA implicit-GEMM
 * convolutions, bandwidth-bound fused epilogues, and a device-resident
 * synthesis session (rvc_synth_*) that has no counterpart in the reference's
 * ABI (its closest analogue is the BatchRunner record/commit path driven from
 * runtime/models/vits.py:676-823, 1165-1253, 1660-1842).
 */
#ifndef RVC_HIP_H
#define RVC_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- engine */
/* replaces rvc_engine_create  (engine/src/ffi.zig:50) */
int64_t rvc_engine_create(void);
/* replaces rvc_engine_destroy (engine/src/ffi.zig:63) */
int32_t rvc_engine_destroy(int64_t h);

/* ---------------------------------------------------------------- memory */
/* replaces rvc_mem_upload       (engine/src/ffi.zig:76): new buffer from n floats */
int32_t rvc_mem_upload(int64_t h, const float* src, int64_t n, int64_t* out_buf);
/* replaces rvc_mem_upload_to    (engine/src/ffi.zig:92): overwrite an existing buffer */
int32_t rvc_mem_upload_to(int64_t h, const float* src, int64_t n, int64_t buf);
/* replaces rvc_mem_upload_bytes (engine/src/ffi.zig:155): raw bytes (int ids, int64 pitch) */
int32_t rvc_mem_upload_bytes(int64_t h, const void* src, int64_t nbytes, int64_t* out_buf);
/* replaces rvc_mem_alloc        (engine/src/ffi.zig:140): uninitialised buffer of nbytes */
int32_t rvc_mem_alloc(int64_t h, int64_t nbytes, int64_t* out_buf);
/* replaces rvc_mem_fill_zero    (engine/src/ffi.zig:170): zero the first nbytes */
int32_t rvc_mem_fill_zero(int64_t h, int64_t buf, int64_t nbytes);
/* replaces rvc_mem_download     (engine/src/ffi.zig:183): copy n floats to host (waits) */
int32_t rvc_mem_download(int64_t h, int64_t buf, float* dst, int64_t n);
/* byte-sized download; no reference counterpart (the reference downloads f32 only) */
int32_t rvc_mem_download_bytes(int64_t h, int64_t buf, void* dst, int64_t nbytes);
/* replaces rvc_mem_free         (engine/src/ffi.zig:222) */
int32_t rvc_mem_free(int64_t h, int64_t buf);
/* replaces rvc_mem_upload_to_batch (engine/src/ffi.zig:107): n uploads into existing buffers,
 * sizes[i] floats from datas[i] into ids[i]; every id and size is checked before any copy */
int32_t rvc_mem_upload_to_batch(int64_t h, int64_t n, const int64_t* sizes, const float* const* datas,
                                const int64_t* ids);
/* replaces rvc_mem_download_batch (engine/src/ffi.zig:199): count downloads, sizes[i] floats of
 * buffer bufs[i] into dsts[i]; one wait at the end */
int32_t rvc_mem_download_batch(int64_t h, const int64_t* bufs, uint8_t* const* dsts, const int64_t* sizes,
                               int64_t count);

/* ---------------------------------------------------------------- single ops */
/* replaces rvc_matmul  (engine/src/ffi.zig:233): c[M,N] = a[M,K] @ b[K,N], row-major */
int32_t rvc_matmul(int64_t h, int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n);
/* replaces rvc_add / rvc_mul (engine/src/ffi.zig:258, :270): c = a (+|*) b over n floats */
int32_t rvc_add(int64_t h, int64_t a, int64_t b, int64_t c, int64_t n);
int32_t rvc_mul(int64_t h, int64_t a, int64_t b, int64_t c, int64_t n);
/* replaces rvc_relu (engine/src/ffi.zig:282): in place */
int32_t rvc_relu(int64_t h, int64_t a, int64_t n);
/* replaces rvc_conv1d (engine/src/ffi.zig:294): x[B,C_in,L], w[C_out,C_in,K], b[C_out] or 0,
 * out[B,C_out,L_out], L_out = (L+pad_l+pad_r-dil*(K-1)-1)/stride+1; bias added in the kernel */
int32_t rvc_conv1d(int64_t h, int64_t x, int64_t w, int64_t b, int64_t out, int64_t B, int64_t c_in,
                   int64_t l, int64_t c_out, int64_t k, int64_t stride, int64_t pad_l, int64_t pad_r,
                   int64_t dil);
/* replaces rvc_conv_t1d (engine/src/ffi.zig:336): w[C_in,C_out,K] (PyTorch ConvTranspose1d layout),
 * L_out = (L-1)*stride - 2*padding + dil*(K-1) + output_padding + 1 */
int32_t rvc_conv_t1d(int64_t h, int64_t x, int64_t w, int64_t b, int64_t out, int64_t B, int64_t c_in,
                     int64_t l, int64_t c_out, int64_t k, int64_t stride, int64_t padding,
                     int64_t output_padding, int64_t dil);
/* No reference counterpart: rvc_conv1d for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same arguments, kernels
 * and results as rvc_conv1d; the weights are packed into a fixed 4 MiB device array per GPU instead of
 * engine scratch, so packed_ld(C_out) * C_in * K (packed_ld = C_out rounded up to 4) must not exceed
 * 1048576 floats, or the call fails with a message.  The call allocates nothing.  Calls on one GPU
 * share the array: calls that overlap on one GPU (several engines' streams at once) race. */
int32_t rvc_conv1d_noalloc(int64_t h, int64_t x, int64_t w, int64_t b, int64_t out, int64_t B, int64_t c_in,
                           int64_t l, int64_t c_out, int64_t k, int64_t stride, int64_t pad_l, int64_t pad_r,
                           int64_t dil);
/* No reference counterpart: rvc_conv1d / rvc_conv_t1d computed on bf16 matrix cores with fp32
 * accumulate (inputs and weights rounded to bf16, nearest even; products summed in fp32), for callers
 * that accept bf16 rounding (the config-5 mixed-precision path).  conv1d: stride 1, K <= 11 and
 * (K-1)*dil <= 64; conv_t1d: dilation 1, stride <= 16 and ceil(K/stride) <= 11.  Same arguments. */
int32_t rvc_conv1d_bf16(int64_t h, int64_t x, int64_t w, int64_t b, int64_t out, int64_t B, int64_t c_in,
                        int64_t l, int64_t c_out, int64_t k, int64_t stride, int64_t pad_l, int64_t pad_r,
                        int64_t dil);
int32_t rvc_conv_t1d_bf16(int64_t h, int64_t x, int64_t w, int64_t b, int64_t out, int64_t B, int64_t c_in,
                          int64_t l, int64_t c_out, int64_t k, int64_t stride, int64_t padding,
                          int64_t output_padding, int64_t dil);
/* replaces rvc_embed (engine/src/ffi.zig:503): out[n,dim] = table[ids[n],:]; ids are int32,
 * validated by the caller (negative ids wrap once) */
int32_t rvc_embed(int64_t h, int64_t ids, int64_t table, int64_t out, int64_t n, int64_t table_rows,
                  int64_t emb_dim);
/* replaces rvc_add_inplace / rvc_mul_inplace (engine/src/ffi.zig:522, :534): a (+|*)= b */
int32_t rvc_add_inplace(int64_t h, int64_t a, int64_t b, int64_t n);
int32_t rvc_mul_inplace(int64_t h, int64_t a, int64_t b, int64_t n);
/* replaces rvc_leaky_relu (engine/src/ffi.zig:549): in place, slope as f32 bits */
int32_t rvc_leaky_relu(int64_t h, int64_t a, int64_t n, int64_t slope);
/* replaces rvc_copy (engine/src/ffi.zig:563): dst != src */
int32_t rvc_copy(int64_t h, int64_t dst, int64_t src, int64_t n);
/* replaces rvc_layernorm (engine/src/ffi.zig:575): row-major [rows, cols], over cols, two-pass */
int32_t rvc_layernorm(int64_t h, int64_t x, int64_t gamma, int64_t beta, int64_t out, int64_t rows,
                      int64_t cols, double eps);
/* replaces rvc_softmax (engine/src/ffi.zig:604): row softmax */
int32_t rvc_softmax(int64_t h, int64_t x, int64_t out, int64_t rows, int64_t cols);
/* replaces rvc_rmsnorm (engine/src/ffi.zig:616): out = x / sqrt(mean(x^2) + eps) * gamma per row */
int32_t rvc_rmsnorm(int64_t h, int64_t x, int64_t gamma, int64_t out, int64_t rows, int64_t cols, double eps);

/* ---------------------------------------------------------------- record / commit */
/* replaces rvc_batch_begin / add / commit / commit_async / wait / discard
 * (engine/src/ffi.zig:880-1017).  Op codes and parameter layout are the
 * reference's (engine/src/ffi.zig:888-929): 1 matmul, 2 conv1d, 3 add_inplace,
 * 4 mul_inplace, 5 conv_t1d, 6 leaky_relu, 7 copy, 8 softmax, 9 layer_norm,
 * 10 gelu, 11 bias_add, 12 attn_qk, 13 attn_sv, 14 relu, 15 group_norm,
 * 16 banded_attn_qk, 17 banded_attn_sv, 18 gating, 19 transpose.  Codes 20-42
 * (training backward ops, 2-D conv, im2col, AdamW scalars) are rejected.
 * Every record is checked when it is added (buffers, sizes, parameters). */
int32_t rvc_batch_begin(int64_t h);
int32_t rvc_batch_add(int64_t h, int32_t op, int64_t a, int64_t b, int64_t c, int64_t p0, int64_t p1,
                      int64_t p2, int64_t p3, int64_t p4, int64_t p5, int64_t p6, int64_t p7, int64_t p8,
                      int64_t p9, int64_t p10);
/* replaces rvc_batch_add_copy_seg (engine/src/ffi.zig:753): dst[a_off..+n) = src[b_off..+n) */
int32_t rvc_batch_add_copy_seg(int64_t h, int64_t a, int64_t b, int64_t n, int64_t a_off, int64_t b_off);
/* replaces rvc_batch_add_add_seg / mul_seg (engine/src/ffi.zig:779, :805): a[a_off..+n) (+|*)= b[b_off..+n) */
int32_t rvc_batch_add_add_seg(int64_t h, int64_t a, int64_t b, int64_t n, int64_t a_off, int64_t b_off);
int32_t rvc_batch_add_mul_seg(int64_t h, int64_t a, int64_t b, int64_t n, int64_t a_off, int64_t b_off);
/* replaces rvc_batch_add_leaky_seg (engine/src/ffi.zig:832): a[a_off..+n) = leaky(a), slope as f32 bits */
int32_t rvc_batch_add_leaky_seg(int64_t h, int64_t a, int64_t n, int64_t a_off, int64_t slope);
/* replaces rvc_batch_add_gelu_seg (engine/src/ffi.zig:858): a[a_off..+n) = gelu(a) (erf form) */
int32_t rvc_batch_add_gelu_seg(int64_t h, int64_t a, int64_t n, int64_t a_off);
/* replaces rvc_batch_add_conv1d_seg (engine/src/ffi.zig:703): a=x b=w c=bias(0=none), p0..p8 as
 * op 2 (pad_r must equal pad_l), p9=out; writes output columns [lo_off, lo_off+seg_len) of the
 * full conv into rows of length l_out_full (lo_off + seg_len <= l_out_full) */
int32_t rvc_batch_add_conv1d_seg(int64_t h, int64_t a, int64_t b, int64_t c, int64_t p0, int64_t p1,
                                 int64_t p2, int64_t p3, int64_t p4, int64_t p5, int64_t p6, int64_t p7,
                                 int64_t p8, int64_t p9, int64_t seg_len, int64_t lo_off, int64_t l_out_full);
/* replaces rvc_batch_add_conv_t1d_seg (engine/src/ffi.zig:636): p0..p8 as op 5, p9=out; output
 * columns [lo_off, lo_off+l_out) into rows of length l_out_full; only input columns
 * [in_off, in_off+l_in_seg) (within the row of length L) contribute; vx/vw/vb/vo are byte offsets
 * of sub-views into x/w/bias/out (-1 = none, else a multiple of 4) */
int32_t rvc_batch_add_conv_t1d_seg(int64_t h, int64_t a, int64_t b, int64_t c, int64_t p0, int64_t p1,
                                   int64_t p2, int64_t p3, int64_t p4, int64_t p5, int64_t p6, int64_t p7,
                                   int64_t p8, int64_t p9, int64_t l_out, int64_t l_in_seg, int64_t in_off,
                                   int64_t lo_off, int64_t l_out_full, int64_t vx, int64_t vw, int64_t vb,
                                   int64_t vo);
int32_t rvc_batch_commit(int64_t h);
int32_t rvc_batch_commit_async(int64_t h);
int32_t rvc_batch_wait(int64_t h);
int32_t rvc_batch_discard(int64_t h);

/* ---------------------------------------------------------------- info */
/* replaces rvc_device_name (engine/src/ffi.zig:1087): needs a live engine */
int32_t rvc_device_name(char* buf, int64_t buf_size);
/* replaces rvc_last_error (engine/src/ffi.zig:1110) */
int32_t rvc_last_error(char* buf, int64_t buf_size);
/* replaces rvc_ts_stats / rvc_ts_reset (engine/src/ffi.zig:1124, :1136): with RVC_TS=1 set when the
 * engine is created, GPU-busy nanoseconds (HIP events around every submission) and the submission
 * count since creation or the last reset; zeros otherwise */
int32_t rvc_ts_stats(int64_t h, int64_t* busy_ns_out, int64_t* submits_out);
int32_t rvc_ts_reset(int64_t h);
/* replaces rvc_mem_stats (engine/src/ffi.zig:1147): every buffer is its own device allocation, so the
 * suballocator / free-list / staging outputs are 0; buf_count, buf_bytes, max_buf_bytes are the live
 * buffers', direct_bytes adds the engine's weight-packing scratch */
int32_t rvc_mem_stats(int64_t h, int64_t* sub_total_out, int64_t* sub_chunks_out, int64_t* sub_free_bytes_out,
                      int64_t* sub_free_blocks_out, int64_t* buf_count_out, int64_t* buf_bytes_out,
                      int64_t* staging_up_out, int64_t* staging_dn_out, int64_t* direct_bytes_out,
                      int64_t* max_buf_bytes_out, int64_t* max_buf_sub_out);
/* replaces rvc_mem_top (engine/src/ffi.zig:1181): the n largest live buffers as (bytes, 0, device
 * address) triples into out[3n]; returns the count written or -1 */
int64_t rvc_mem_top(int64_t h, int64_t n, int64_t* out);
/* replaces rvc_probe_extensions (engine/src/ffi.zig:1426): "shaderFloat16=1,VK_KHR_cooperative_matrix=1,
 * VK_KHR_shader_float16_int8=1,arch=<gfx name>" (the capabilities those flags stand for, on the HIP
 * device), NUL-terminated; -1 if buf_size is too small */
int32_t rvc_probe_extensions(int64_t h, char* buf, int64_t buf_size);

/* ---------------------------------------------------------------- RMVPE ops
 * rvc_conv2d (engine/src/ffi.zig:378): out[B][C_out][OH][OW] = conv2d(x[B][C_in]
 * [ih][iw], w[C_out][C_in][kh][kw]) + b (b == 0: none), symmetric padding,
 * dilation 1; on this backend kh, kw <= 3 and stride_h == stride_w in {1, 2}
 * (RMVPE's 3x3 / 1x1 convs and the 2x2 stride-2 pooling conv), other shapes
 * return -1 with a message.
 * rvc_gru (ffi.zig:1394, engine.zig:3097): bidirectional GRU recurrence, a =
 * gate inputs [2T][3H] (forward rows then reverse rows, time order), b = W_hh
 * [2][3H][H], c = b_hh [2][3H], out [T][2H]; H <= 256. */
int32_t rvc_conv2d(int64_t h, int64_t x, int64_t w, int64_t b, int64_t out, int64_t B, int64_t c_in, int64_t ih,
                   int64_t iw, int64_t c_out, int64_t kh, int64_t kw, int64_t pad_h, int64_t pad_w, int64_t stride_h,
                   int64_t stride_w);
int32_t rvc_gru(int64_t h, int64_t a, int64_t b, int64_t c, int64_t out, int64_t t, int64_t hdim);
/* rvc_conv_t2d (ffi.zig:428, engine.zig:1511): out[B][C_out][h_out][w_out] =
 * conv_transpose2d(x[B][C_in][ih][iw], w[C_in][C_out][kh][kw]), stride (sh, sw),
 * padding (ph, pw), output padding < stride, no bias; h_out / w_out must match
 * the transposed-conv formula; kh, kw <= 3 and sh, sw <= 2 on this backend.
 * rvc_insert_zeros_2x (ffi.zig:481, engine.zig:1704): out[C][2H-1][2W-1] = x at
 * even rows and columns, zeros elsewhere (RMVPE's zero-inserted ConvTranspose
 * input, fed to rvc_conv2d). */
int32_t rvc_conv_t2d(int64_t h, int64_t x, int64_t w, int64_t out, int64_t B, int64_t c_in, int64_t ih, int64_t iw,
                     int64_t c_out, int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                     int64_t opad_h, int64_t opad_w, int64_t h_out, int64_t w_out);
int32_t rvc_insert_zeros_2x(int64_t h, int64_t x, int64_t out, int64_t c, int64_t ih, int64_t iw);
/* Record/commit forms (ffi.zig:1196 rvc_batch_add_conv2d, :1246
 * rvc_batch_add_conv_t2d, :1377 rvc_batch_add_gru): the same ops appended to
 * the pending batch and run in order by rvc_batch_commit /
 * rvc_batch_commit_async.  rvc_batch_add_conv_t2d takes a bias b (0: none).
 * Arguments are checked when recorded; a GRU whose step barrier gave up is
 * reported by rvc_batch_commit / rvc_batch_wait. */
int32_t rvc_batch_add_conv2d(int64_t h, int64_t x, int64_t w, int64_t b, int64_t out, int64_t B, int64_t c_in,
                             int64_t ih, int64_t iw, int64_t c_out, int64_t kh, int64_t kw, int64_t pad_h,
                             int64_t pad_w, int64_t stride_h, int64_t stride_w);
int32_t rvc_batch_add_conv_t2d(int64_t h, int64_t x, int64_t w, int64_t b, int64_t out, int64_t B, int64_t c_in,
                               int64_t ih, int64_t iw, int64_t c_out, int64_t kh, int64_t kw, int64_t sh,
                               int64_t sw, int64_t ph, int64_t pw, int64_t opad_h, int64_t opad_w, int64_t h_out,
                               int64_t w_out);
int32_t rvc_batch_add_gru(int64_t h, int64_t a, int64_t b, int64_t c, int64_t out, int64_t t, int64_t hdim);

/* ---------------------------------------------------------------- not provided
 * Exported so the reference's loader (runtime/_vulkan.py:148-278 binds every
 * symbol) can load this library; each returns -1 with a message.  They serve
 * training and the reference's record/commit form of the RMVPE ops:
 * rvc_matmul_f16 (ffi.zig:246), rvc_batch_add_im2col_1d (:1304),
 * rvc_batch_add_im2col_2d (:1341) and the barrier-only GRU diagnostic
 * rvc_batch_add_gru_sync (:1411); the 2-D convs here are implicit GEMMs that
 * need no im2col buffer.  RMVPE as a whole runs in the rvc_rmvpe_* session
 * below. */
int32_t rvc_matmul_f16(int64_t h, int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n);
int32_t rvc_batch_add_im2col_1d(int64_t h, int64_t x, int64_t out, int64_t B, int64_t c, int64_t t, int64_t o_l,
                                int64_t k_dil, int64_t stride, int64_t pad_l, int64_t dilation);
int32_t rvc_batch_add_im2col_2d(int64_t h, int64_t x, int64_t out, int64_t B, int64_t c, int64_t ih, int64_t iw,
                                int64_t oh, int64_t ow, int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph,
                                int64_t pw);
int32_t rvc_batch_add_gru_sync(int64_t h, int64_t a, int64_t t, int64_t hdim);

/* ---------------------------------------------------------------- synthesis session
 * No counterpart in the reference ABI.  A session owns device-resident,
 * pre-packed weights of one RVC v2 synthesizer and runs
 * SynthesizerTrn.infer_controlled (runtime/models/vits.py:2551-2595) or
 * _GeneratorNSF.forward (runtime/models/vits.py:2133-2231) as one stream of
 * fused HIP kernels.  Tensors are float32, batch-major; B independent
 * chunks of P frames each. */
int64_t rvc_synth_create(int64_t h);
int32_t rvc_synth_destroy(int64_t s);
/* Register one checkpoint tensor by its RVC key (e.g. "dec.ups.0.weight_v");
 * weight-norm pairs are resolved at finalize (runtime/models/vits.py:416-442). */
int32_t rvc_synth_set_weight(int64_t s, const char* key, const float* data, const int64_t* shape,
                             int32_t ndim);
/* Derive the geometry from the registered shapes plus the upsample rates /
 * kernels and the sample rate (VitsConfig, runtime/models/vits.py:166-268),
 * pack and upload every weight. */
int32_t rvc_synth_finalize(int64_t s, int64_t sr, const int64_t* rates, const int64_t* kernels,
                           int32_t n_ups);
/* Host in -> host out.  phone [B,P,phone_dim], pitch int64 [B,P], nsff0 [B,P],
 * sid int64 [B], nz [B,hidden,P], ns [B,P*upp] -> wave [B,P*upp]. */
int32_t rvc_synth_infer(int64_t s, const float* phone, const int64_t* pitch, const float* nsff0,
                        const int64_t* sid, const float* nz, const float* ns, int64_t B, int64_t P,
                        float* wave);
/* Deferred form of rvc_synth_infer (SynthesizerTrn.infer(..., phone_gpu=...,
 * _defer=True), runtime/models/vits.py:2352-2402, 2551-2595, used by
 * Pipeline's chunk overlap, runtime/pipeline.py:1010-1080): queue the whole
 * synthesis and the waveform's copy into pinned staging, return a ticket
 * (> 0) without waiting, -1 on error.  phone is a host [B,P,phone_dim] array,
 * or 0 with phone_buf the engine buffer holding it (the resident phone_gpu);
 * exactly one of them.  Host arrays may be reused once the call returns.
 * At most 8 calls are outstanding per session; each is ended by
 * rvc_synth_collect (waits, copies the wave [B,P*upp] out) or
 * rvc_synth_abort (waits, drops it).  Calls run in submission order. */
int64_t rvc_synth_submit(int64_t s, const float* phone, int64_t phone_buf, const int64_t* pitch,
                         const float* nsff0, const int64_t* sid, const float* nz, const float* ns, int64_t B,
                         int64_t P);
int32_t rvc_synth_collect(int64_t s, int64_t ticket, float* wave);
int32_t rvc_synth_abort(int64_t s, int64_t ticket);
/* Same with engine buffer ids (inputs already resident; pitch/sid hold int64).
 * A pitch or sid id outside [-rows, rows) fails the call (-1, "... out of
 * range"), as the host path and numpy's take do. */
int32_t rvc_synth_infer_dev(int64_t s, int64_t phone, int64_t pitch, int64_t nsff0, int64_t sid,
                            int64_t nz, int64_t ns, int64_t B, int64_t P, int64_t wave);
/* enc_p + flow without the decoder: SynthesizerTrn._full_prep (flow_head = 0)
 * and the enc_p/flow half of _partial_prep (runtime/models/vits.py:2416-2500):
 * enc_p over all P frames, z_p = m + exp(logs)*nz*0.66666, the flow over
 * frames [flow_head, P).  z_out [B,hidden,P-flow_head]; g_out [B,gin]
 * (nullable); phase_out [B,P] (nullable, needs nsff0 [B,P]) receives
 * _phase_offsets(nsff0) = fmod(cumsum(fmod(f0/sr*upp + 0.5, 1) - 0.5), 1)
 * (:2404-2414). */
int32_t rvc_synth_prep(int64_t s, const float* phone, const int64_t* pitch, const float* nsff0,
                       const int64_t* sid, const float* nz, int64_t B, int64_t P, int64_t flow_head,
                       float* z_out, float* g_out, float* phase_out);
/* SynthesizerTrn._phase_offsets (runtime/models/vits.py:2404-2414) of nsff0
 * [B,P]: out [B,P] = fmod(cumsum(fmod(f0/sr*upp + 0.5, 1) - 0.5), 1), the
 * cumulative sum taken sequentially in float32. */
int32_t rvc_synth_phase_offsets(int64_t s, const float* nsff0, int64_t B, int64_t P, float* out);
/* Decoder only: z [B,hidden,P], f0 [B,P], g [B,gin], ns [B,P*upp] -> wave [B,P*upp]. */
int32_t rvc_synth_decode(int64_t s, const float* z, const float* f0, const float* g, const float* ns,
                         int64_t B, int64_t P, float* wave);
int32_t rvc_synth_decode_dev(int64_t s, int64_t z, int64_t f0, int64_t g, int64_t ns, int64_t B,
                             int64_t P, int64_t wave);
/* _GeneratorNSF.decode_batch (runtime/models/vits.py:1847-1878): n chunks of
 * P[i] frames each, z[i] [hidden,P[i]], f0[i] [P[i]], ns[i] [P[i]*upp], off[i]
 * [P[i]] (the per-frame phase offsets seg_offsets, :1484-1491; off or off[i]
 * may be null for f0's own cumulative phase), one speaker g [gin] (null: no
 * speaker term) -> wave[i] [P[i]*upp].  Chunks of equal length run as one
 * batch and the batches follow each other on one stream; each result equals
 * that chunk's own decode bit for bit. */
int32_t rvc_synth_decode_chunks(int64_t s, int64_t n, const float* const* z, const float* const* f0,
                                const float* const* ns, const float* const* off, const int64_t* P,
                                const float* g, float* const* wave);
/* Copy a named intermediate of the last run to the host (n floats): "enc_in",
 * "enc_out", "stats", "z_p", "z", "g", "har", "dec_pre", "dec_stage0".."dec_stage3". */
int32_t rvc_synth_read(int64_t s, const char* name, float* dst, int64_t n);
/* Before rvc_synth_finalize: 0 = fp32 (default); 1 = the GeneratorNSF upsample ConvTranspose1d and
 * the enc_p matmuls (embedding linear, q/k/v, conv_o, FFN, proj) on bf16 MFMA with fp32 accumulate
 * (BASELINE config 5); 2 = mode 1 plus the decoder ResBlock convs on bf16. */
int32_t rvc_synth_set_precision(int64_t s, int32_t mode);
/* Keep a copy of each decoder stage output ("dec_stage<i>") for rvc_synth_read. */
int32_t rvc_synth_set_debug(int64_t s, int32_t keep_stages);
/* Per-kernel-family timing with HIP events on the session stream.  tag selects
 * the launches to time (prefix match, e.g. "dec.rb.s1"); "" disables. */
int32_t rvc_synth_set_timing(int64_t s, const char* tag);
int32_t rvc_synth_get_timing(int64_t s, double* total_ms, int64_t* launches, double* flops, double* bytes);

/* ---------------------------------------------------------------- HuBERT session
 * No counterpart in the reference ABI.  A device-resident HuBERT-base encoder:
 * HubertEncoder.encode (runtime/models/hubert.py:564-591) as one stream of HIP
 * kernels over weights uploaded once.  Weights are registered under their
 * transformers state-dict keys (runtime/models/hubert.py:524-558); the
 * positional conv's weight norm is resolved at finalize (:510-522). */
int64_t rvc_hubert_create(int64_t h);
int32_t rvc_hubert_destroy(int64_t s);
int32_t rvc_hubert_set_weight(int64_t s, const char* key, const float* data, const int64_t* shape, int32_t ndim);
int32_t rvc_hubert_finalize(int64_t s);
/* Output frames L of the feature extractor for T input samples. */
int32_t rvc_hubert_frames(int64_t s, int64_t T, int64_t* L);
/* x [B,T] float32 16 kHz -> out [B,L,768] (version 2, last hidden state) or
 * [B,L,256] (version 1, final_proj of layer 9). */
int32_t rvc_hubert_encode(int64_t s, const float* x, int64_t B, int64_t T, int32_t version, float* out);
int32_t rvc_hubert_encode_dev(int64_t s, int64_t x, int64_t B, int64_t T, int32_t version, int64_t out);
/* Named intermediates of the last call, channel-major [B,C,L]: "feats",
 * "proj", "pos", "entry", and "layer1" after rvc_hubert_set_debug(s, 1). */
int32_t rvc_hubert_read(int64_t s, const char* name, float* dst, int64_t n);
int32_t rvc_hubert_set_debug(int64_t s, int32_t keep);
int32_t rvc_hubert_set_timing(int64_t s, const char* tag);
int32_t rvc_hubert_get_timing(int64_t s, double* total_ms, int64_t* launches, double* flops, double* bytes);

/* ---------------------------------------------------------------- RMVPE session
 * No counterpart in the reference ABI.  A device-resident RMVPE pitch
 * extractor: RMVPE.infer_from_audio (runtime/models/rmvpe.py:927-952) -- log-mel
 * front end (:632-640), the U-Net of ConvBlockRes levels (:643-690), cnn, BiGRU,
 * Linear + sigmoid (:727-751) and the local-average cents decode (:899-924) --
 * as one stream of HIP kernels over weights uploaded once.  Weights are
 * registered under the rmvpe.pt state-dict keys; BatchNorm is folded into the
 * convolutions at finalize. */
int64_t rvc_rmvpe_create(int64_t h);
int32_t rvc_rmvpe_destroy(int64_t r);
int32_t rvc_rmvpe_set_weight(int64_t r, const char* key, const float* data, const int64_t* shape, int32_t ndim);
int32_t rvc_rmvpe_finalize(int64_t r);
/* STFT frames F = 1 + T / 160 for T samples (runtime/dsp/fft.py:102). */
int32_t rvc_rmvpe_frames(int64_t r, int64_t T, int64_t* F);
/* audio [T] float32 16 kHz (T > 512) -> f0 [F] Hz, 0 where the salience
 * maximum is <= thred (infer_from_audio(x, thred)). */
int32_t rvc_rmvpe_infer(int64_t r, const float* x, int64_t T, double thred, float* f0);
int32_t rvc_rmvpe_infer_dev(int64_t r, int64_t x, int64_t T, double thred, int64_t f0);
/* Named intermediates of the last call: "mel" [128][F] log-mel, "salience"
 * [360][F'] (F' = F rounded up to a multiple of 32; mel2hidden is its
 * transpose cut to F frames), "gru_in" [384][F'], "gru_out" [512][F']. */
int32_t rvc_rmvpe_read(int64_t r, const char* name, float* dst, int64_t n);
int32_t rvc_rmvpe_set_timing(int64_t r, const char* tag);
int32_t rvc_rmvpe_get_timing(int64_t r, double* total_ms, int64_t* launches, double* flops, double* bytes);

/* ---------------------------------------------------------------- conversion glue session
 * No counterpart in the reference ABI.  The steps of runtime/pipeline.py either
 * side of SynthesizerTrn.infer, on device: feature retrieval against a resident
 * index (search_l2, runtime/retrieval.py:35-83, and the blend of
 * runtime/pipeline.py:546-566), the 2x feature interpolation and pitch protect
 * mask (runtime/pipeline.py:568-610, runtime/nn.py:734-758), the RMS envelope
 * mix (change_rms, runtime/pipeline.py:164-232) and the int16 peak
 * normalisation (runtime/pipeline.py:1208-1213).  Features are row-major
 * [F, D] (the HuBERT output layout). */
int64_t rvc_vc_create(int64_t h);
int32_t rvc_vc_destroy(int64_t v);
/* Make vectors [n, dim] the resident retrieval index (FeatureIndex.add +
 * reconstruct_n, runtime/retrieval.py:113-140); replaces any previous one. */
int32_t rvc_vc_set_index(int64_t v, const float* vectors, int64_t n, int64_t dim);
int32_t rvc_vc_index_info(int64_t v, int64_t* n, int64_t* dim);
/* search_l2 (runtime/retrieval.py:35-83): the k (1..min(8, n)) nearest index
 * rows of each query row, squared L2 distances ascending (clamped at 0) and
 * int64 row numbers; equal distances keep the lower row first. */
int32_t rvc_vc_search(int64_t v, const float* query, int64_t F, int64_t k, float* scores, int64_t* inds);
int32_t rvc_vc_search_dev(int64_t v, int64_t query, int64_t F, int64_t k, int64_t scores, int64_t inds);
/* Pipeline._vc_prepare's feature path (runtime/pipeline.py:488-614, FeatureIndex
 * branch): when index_rate != 0 and an index is set, feats = blend * index_rate
 * + feats * (1 - index_rate) with blend the (1/d)^2-weighted mean of the 8
 * nearest index rows; then 2x linear interpolation to [2F, D]; then, when
 * pitchf [2F] (already aligned to 2F frames) is given, the protect mask
 * out = feats * pff + feats0 * (1 - pff), pff = 1 where pitchf > 0, protect
 * where pitchf < 1, feats0 the interpolated features before retrieval.
 * pitchf null (or buffer 0): no protect mask (protect >= 0.5 in the reference). */
int32_t rvc_vc_prepare(int64_t v, const float* feats, int64_t F, int64_t D, double index_rate,
                       const float* pitchf, double protect, float* out);
int32_t rvc_vc_prepare_dev(int64_t v, int64_t feats, int64_t F, int64_t D, double index_rate, int64_t pitchf,
                           double protect, int64_t out);
/* change_rms(data1, data2, sr1, sr2, rate) (runtime/pipeline.py:164-188):
 * data2 * rms1^(1-rate) * max(rms2, 1e-6)^(rate-1), the half-second frame RMS
 * curves linearly interpolated to n2 samples. */
int32_t rvc_vc_change_rms(int64_t v, const float* data1, int64_t n1, int64_t sr1, const float* data2, int64_t n2,
                          int64_t sr2, double rate, float* out);
int32_t rvc_vc_change_rms_dev(int64_t v, int64_t data1, int64_t n1, int64_t sr1, int64_t data2, int64_t n2,
                              int64_t sr2, double rate, int64_t out);
/* int16(x * 32768 / max(1, max|x| / 0.99)) (runtime/pipeline.py:1208-1213). */
int32_t rvc_vc_to_int16(int64_t v, const float* x, int64_t n, int16_t* out);
int32_t rvc_vc_to_int16_dev(int64_t v, int64_t x, int64_t n, int64_t out);
int32_t rvc_vc_set_timing(int64_t v, const char* tag);
int32_t rvc_vc_get_timing(int64_t v, double* total_ms, int64_t* launches, double* flops, double* bytes);

#ifdef __cplusplus
}
#endif

#endif /* RVC_HIP_H */
