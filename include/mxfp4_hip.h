/* mxfp4_hip.h -- C ABI of the MI355X (gfx950) MXFP4 MoE hot path.
 *
 * Plain C: device pointers, sizes and a HIP stream passed as void*
 * (a hipStream_t; NULL = the default stream).  No torch types.  Every entry
 * point validates its arguments on the host, launches asynchronously on the
 * given stream, and returns MXFP4_OK (0), MXFP4_EINVAL (-1, see
 * mxfp4_last_error()) or a positive hipError_t from the launch.
 *
 * Data formats (unchanged from the reference, quant/quantize_mxfp4.py:110-160):
 *   packed MXFP4 rows  u8 (rows, Kp/2): two E2M1 nibbles per byte, element 2j
 *                      in the low nibble (quant/fp4_format.py:126-137);
 *   scale codes        u8 (rows, Kp/32): E8M0, value 2^(code-127);
 *   Kp = ceil(K/32)*32, padding elements are zero.
 * Quantization is bit-exact to quant/fp4_format.py (E2M1 ties to the larger
 * magnitude; smallest power-of-two scale with amax/scale <= 6).
 */
#ifndef MXFP4_HIP_H
#define MXFP4_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MXFP4_HIP_ABI_VERSION 1

enum {
    MXFP4_OK = 0,
    MXFP4_EINVAL = -1,   /* argument check failed; message in mxfp4_last_error() */
    MXFP4_ETIMEOUT = -2  /* a fused kernel's bounded wait expired (see mxfp4_decode_layer_status) */
};

/* Activation dtypes accepted by the quantizers. */
enum { MXFP4_DT_BF16 = 0, MXFP4_DT_F16 = 1, MXFP4_DT_F32 = 2 };

/* Largest pointer table passed by value to one grouped launch; longer tables
 * are processed in several launches. */
#define MXFP4_MAX_TABLE 160

int mxfp4_abi_version(void);
/* Message of the last MXFP4_EINVAL on the calling thread ("" if none). */
const char* mxfp4_last_error(void);

/* ---------------------------------------------------------------------
 * Activation quantizer.
 * Replaces mxfp4v2::launch_prequant_v2 (src/ext/mxfp4_decode.cu:304-309),
 * bound as `prequant` (src/ext/mxfp4_decode_binding.cpp:65-81).
 * x: bf16 (M, K) with row stride ldx elements; writes every byte of
 * xq (M, Kp/2) and xsc (M, Kp/32).  Kp must be a multiple of 32 and >= K.
 * Unlike src/ext/mxfp4_decode.cu:46 the last element of an odd K is packed
 * (quant/fp4_format.py contract).
 */
int mxfp4_prequant(const void* x, int64_t ldx, int M, int K, int Kp,
                   uint8_t* xq, uint8_t* xsc, void* stream);

/* Same quantizer for bf16 / fp16 / fp32 rows (src_dtype = MXFP4_DT_*).
 * round_to_f16 = 1: each element is first rounded to fp16, as the
 * reference's `forward` does (src/ext/mxfp4_binding.cpp:31); 2: first
 * rounded to bf16 (an fp32 tensor's `.to(torch.bfloat16)` before prequant,
 * runtime/model_runner_v2.py:262-263); 0: as is. */
int mxfp4_quantize_rows(const void* x, int src_dtype, int round_to_f16, int64_t ldx,
                        int M, int K, int Kp, uint8_t* q, uint8_t* s, void* stream);

/* ---------------------------------------------------------------------
 * Block-scaled GEMM on pre-quantized activations: y (M, N) fp32 = A_q * W_q^T.
 * Replaces mxfp4v2::launch_lin_pq_v2 (src/ext/mxfp4_decode.cu:311-318),
 * bound as `lin_pq` (src/ext/mxfp4_decode_binding.cpp:84-98).
 * xq (M, Kp/2), xsc (M, Kp/32), wp (N, Kp/2), wsc (N, Kp/32).  The sum runs
 * over all Kp (activation padding must be zero nibbles, as prequant writes).
 */
int mxfp4_lin_pq(const uint8_t* xq, const uint8_t* xsc, const uint8_t* wp,
                 const uint8_t* wsc, float* y, int M, int N, int K, int Kp,
                 void* stream);

/* ---------------------------------------------------------------------
 * Linear with on-the-fly activation quantization: y (M, N) fp32.
 * Replaces mxfp4::launch_mxfp4_linear (src/ext/mxfp4_linear.cu:200-206),
 * bound as `forward` (src/ext/mxfp4_binding.cpp:21-45).
 * x (M, K) bf16 or fp16 (x_dtype), contiguous.  Activations are rounded to
 * fp16 first (src/ext/mxfp4_binding.cpp:31), then quantized per 32-block over
 * the weight's Kp into `workspace` (>= mxfp4_linear_workspace_size bytes,
 * device memory), then multiplied.
 */
size_t mxfp4_linear_workspace_size(int M, int Kp);
int mxfp4_linear_forward(const void* x, int x_dtype, const uint8_t* wp,
                         const uint8_t* wsc, float* y, int M, int N, int K, int Kp,
                         void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------
 * Grouped gate/up projection over a token-major pointer table.
 * Replaces mxfp4v2::launch_gateup_v2 (src/ext/mxfp4_decode.cu:320-328),
 * bound as `moe_gateup` (src/ext/mxfp4_decode_binding.cpp:101-120).
 * Table entry t = m*2E + proj*E + e (runtime/model_runner_v2.py:279-286)
 * holds the weight (N, Kp/2) + scales (N, Kp/32) applied to activation row
 * m of xq/xsc; the result goes to gu[(m*E+e)*2N + proj*N + n] (fp32,
 * (M*E, 2N)).  Entries with identical weight pointers share one pass over
 * the weight.  The tables are host arrays of 2*E*M device pointers; they are
 * passed by value in kernel arguments (no host-blocking copy, unlike
 * src/ext/mxfp4_decode_binding.cpp:44-60).
 */
int mxfp4_moe_gateup(const uint8_t* xq, const uint8_t* xsc,
                     const uint8_t* const* wp_tab, const uint8_t* const* wsc_tab,
                     float* gu, int E, int M, int N, int K, int Kp, void* stream);

/* As mxfp4_moe_gateup with the tables in device memory (int64 pointers),
 * bound as `moe_gateup_tab` (src/ext/mxfp4_decode_binding.cpp:177-192). */
int mxfp4_moe_gateup_devtab(const uint8_t* xq, const uint8_t* xsc,
                            const int64_t* wp_tab, const int64_t* wsc_tab,
                            float* gu, int E, int M, int N, int K, int Kp, void* stream);

/* ---------------------------------------------------------------------
 * Fused SiLU-gate + MXFP4 re-quantization + down projection.
 * Replaces mxfp4v2::launch_down_silu_v2 (src/ext/mxfp4_decode.cu:330-338),
 * bound as `moe_down` (src/ext/mxfp4_decode_binding.cpp:123-142).
 * For row z = m*E+e of gu (M*E, 2K): h = g/(1+exp(-g))*u in fp32 with
 * g = gu[z, 0:K], u = gu[z, K:2K]; h is quantized per 32-block (zero past
 * K) and multiplied with table entry z (N, Kp/2); yd (M*E, N) fp32.
 */
int mxfp4_moe_down(const float* gu, const uint8_t* const* wp_tab,
                   const uint8_t* const* wsc_tab, float* yd, int E, int M, int N,
                   int K, int Kp, void* stream);

/* As mxfp4_moe_down with device tables, bound as `moe_down_tab`
 * (src/ext/mxfp4_decode_binding.cpp:194-209). */
int mxfp4_moe_down_devtab(const float* gu, const int64_t* wp_tab, const int64_t* wsc_tab,
                          float* yd, int E, int M, int N, int K, int Kp, void* stream);

/* ---------------------------------------------------------------------
 * Weighted top-k combine: out[m, c] = sum_{e < min(E, 8)} w[m, e] * yd[m*E+e, c].
 * Replaces mxfp4v2::launch_combine_v2 (src/ext/mxfp4_decode.cu:340-344),
 * bound as `moe_combine` (src/ext/mxfp4_decode_binding.cpp:145-158).  Slots
 * past 8 are ignored exactly as the reference does (src/ext/mxfp4_decode.cu:296).
 */
int mxfp4_moe_combine(const float* yd, int ystride, const float* w, int E,
                      float* out, int M, int N, void* stream);

/* ---------------------------------------------------------------------
 * Decode attention over one layer's FP8 KV cache.
 * Replaces mxfp4v2::launch_attn_decode_v2 (src/ext/mxfp4_decode.cu:366-430),
 * bound as `attn_decode` (src/ext/mxfp4_decode_binding.cpp:213-230).
 *   q          bf16 (M, Hq, D), D = 128, Hq = G*Hkv with G in {1,2,4,8,16}
 *   kvk/kvv    cache bytes (max_pos, Hkv, D) in the reference's E4M3 codec
 *              (kvk 16-byte aligned)
 *   dpos       device int32: base position; token m sits at dpos+m and
 *              attends to positions 0..dpos+m (rows outside [0, max_pos)
 *              are skipped, as in the reference); read on the device, so a
 *              captured graph follows updates of it
 *   sc         f32 (M, Hq, max_pos) scratch; receives the raw scores q.k
 *   o          f32 (M, Hq, D): softmax(q.k / sqrt(D)) . v
 *   workspace  16-byte aligned device memory of
 *              mxfp4_attn_decode_workspace_size(M, Hq, max_pos) bytes (the
 *              per-64-position softmax partials; nothing persists)
 */
size_t mxfp4_attn_decode_workspace_size(int M, int Hq, int max_pos);
int mxfp4_attn_decode(const void* q, const uint8_t* kvk, const uint8_t* kvv, const int32_t* dpos,
                      float* sc, float* o, int M, int Hq, int Hkv, int D, int max_pos,
                      void* workspace, size_t workspace_bytes, void* stream);

/* mxfp4_attn_decode_mx: mxfp4_attn_decode whose output can also (or only)
 * be the MXFP4 rows of bf16(o), the activation of the o_proj lin_pq
 * (runtime/model_runner_v2.py:175-178: o.bfloat16() -> prequant): oq u8
 * (M, Hq*D/2) and os u8 (M, Hq*D/32), bit-exact to mxfp4_quantize_rows of
 * o with bf16 rounding (mode 2).  o may be NULL when oq/os are given, and
 * sc may be NULL (the raw scores are then not kept: a caller that never
 * reads them saves M*Hq*(dpos+M) four-byte stores). */
int mxfp4_attn_decode_mx(const void* q, const uint8_t* kvk, const uint8_t* kvv, const int32_t* dpos,
                         float* sc, float* o, uint8_t* oq, uint8_t* os, int M, int Hq, int Hkv, int D,
                         int max_pos, void* workspace, size_t workspace_bytes, void* stream);

/* mxfp4_attn_decode_fused: mxfp4_qk_norm_rope_kv followed by
 * mxfp4_attn_decode_mx in one pass over the cache, bit-exact to that pair
 * (same q, cache bytes, sc and outputs): qkv fp32 (M, (Hq + 2 Hkv) * D) are
 * the step's projections, the q heads are normalised and rotated inside the
 * attention kernel and the step's k / v rows (positions *dpos .. *dpos+M-1)
 * are encoded there, used for the scores and written to kvk / kvv.  It has
 * no single counterpart in the reference, whose step runs q_norm / k_norm /
 * RoPE (runtime/model_runner_v2.py:155-163), kv_write and attn_decode
 * (src/ext/mxfp4_decode.cu:352-490) as separate launches; it saves a launch
 * and a memory round trip per layer.  M <= 16, D = 128; codec as
 * mxfp4_qk_norm_rope_kv; workspace as mxfp4_attn_decode; o and sc may be
 * NULL as for mxfp4_attn_decode_mx. */
int mxfp4_attn_decode_fused(const float* qkv, const void* q_norm_w, const void* k_norm_w, float eps,
                            float theta, uint8_t* kvk, uint8_t* kvv, const int32_t* dpos, float* sc, float* o,
                            uint8_t* oq, uint8_t* os, int M, int Hq, int Hkv, int D, int max_pos, int codec,
                            void* workspace, size_t workspace_bytes, void* stream);

/* mxfp4_attn_decode_fused_partials: the first pass of mxfp4_attn_decode_fused
 * alone -- q/k norm, RoPE, the KV write and every 64-position chunk's softmax
 * record -- leaving the records in the workspace for the merge that
 * mxfp4_decode_layer_post_attn runs at the front of the MoE launch (no merge
 * launch here).  Arguments as mxfp4_attn_decode_fused without outputs. */
int mxfp4_attn_decode_fused_partials(const float* qkv, const void* q_norm_w, const void* k_norm_w, float eps,
                                     float theta, uint8_t* kvk, uint8_t* kvv, const int32_t* dpos, int M, int Hq,
                                     int Hkv, int D, int max_pos, int codec, void* workspace,
                                     size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------
 * KV write: k, v bf16 (M, Hkv, D) -> the reference's E4M3 bytes (rounding
 * half away from zero, >= 248 saturating to 0x7F) at rows dpos+m < max_pos
 * of kvk / kvv (max_pos, Hkv, D); nothing when dpos < 0.
 * Replaces mxfp4v2::launch_kvwrite_v2 (src/ext/mxfp4_decode.cu:437-489),
 * bound as `kv_write` (src/ext/mxfp4_decode_binding.cpp:161-173).
 */
int mxfp4_kv_write(const void* k, const void* v, uint8_t* kvk, uint8_t* kvv, const int32_t* dpos,
                   int M, int Hkv, int D, int max_pos, void* stream);

/* ---------------------------------------------------------------------
 * Fused decode MoE layer, one launch per layer, batch 1.
 * Replaces the per-layer sequence prequant -> moe_gateup -> moe_down ->
 * moe_combine -> `x + moe.bfloat16()` of runtime/model_runner_v2.py:185-208
 * for one token, computed on the UN-quantized bf16 activations (the
 * dequant-to-BF16 path of runtime/model_runner.py:128-131 in fp32).
 *   x          bf16 (H), 16-byte aligned
 *   routing    E expert ids + E combine weights (runtime/model_runner_v2.py:
 *              189-192), either by value from the host (ids_host/w_host,
 *              ids_dev = w_dev = NULL) or in device memory (ids_dev/w_dev)
 *   weights    per layer, the n_experts experts stacked back to back, each
 *              in the reference layout: gate/up (Mi, H/2) + (Mi, H/32),
 *              down (H, Mi/2) + (H, Mi/32)
 *   out        fp32 (H): sum_e w_e * down_e(silu(gate_e x) * up_e x)
 *   resid_out  optional bf16 (H): bf16(x + bf16(out)), or NULL
 *   workspace  device memory of mxfp4_decode_layer_workspace_size(E, Mi)
 *              bytes (~53 KB at E=8, Mi=768), 256-byte aligned, initialised
 *              once by mxfp4_decode_layer_reset(workspace, E, H, Mi); every
 *              launch leaves it ready for the next one, so it needs no reset
 *              between launches or HIP graph replays.  Every launch on it
 *              must use that (E, H, Mi) (a launch with another shape sets the
 *              error flag instead of waiting); launches sharing a workspace
 *              must be stream-ordered.
 * Limits: E <= 8, H a multiple of 512 up to 2048, Mi a multiple of 32 up to
 * 1024.  Returns MXFP4_OK or an error; a bounded internal wait that expired
 * is reported by mxfp4_decode_layer_status (the flag stays set; reset the
 * workspace before launching on it again).
 */
size_t mxfp4_decode_layer_workspace_size(int E, int Mi);
int mxfp4_decode_layer_reset(void* workspace, int E, int H, int Mi, void* stream);
int mxfp4_decode_layer_status(const void* workspace, int* error_flag);
int mxfp4_moe_decode_layer(const void* x, const int32_t* ids_host, const float* w_host,
                           const int32_t* ids_dev, const float* w_dev,
                           const uint8_t* gate_wp, const uint8_t* gate_ws,
                           const uint8_t* up_wp, const uint8_t* up_ws,
                           const uint8_t* down_wp, const uint8_t* down_ws,
                           int n_experts, int E, int H, int Mi, float* out, void* resid_out,
                           void* workspace, size_t workspace_bytes, void* stream);

/* As mxfp4_moe_decode_layer with the routing computed in the same launch
 * from the layer's router logits (runtime/model_runner_v2.py:189-192:
 * softmax over n_experts fp32 logits, top-E, renormalised when norm), the
 * same rule and ids as mxfp4_route_topk.  Every workgroup derives the E
 * (id, weight) pairs itself, so the step needs no separate routing launch and
 * no host round trip.  logits: fp32 (n_experts) in device memory,
 * n_experts <= 256.  ids_out / w_out: optional int32 / fp32 (E) device
 * arrays receiving the routing (both or neither).
 */
int mxfp4_moe_decode_layer_routed(const void* x, const float* logits, int norm, int32_t* ids_out,
                                  float* w_out, const uint8_t* gate_wp, const uint8_t* gate_ws,
                                  const uint8_t* up_wp, const uint8_t* up_ws, const uint8_t* down_wp,
                                  const uint8_t* down_ws, int n_experts, int E, int H, int Mi,
                                  float* out, void* resid_out, void* workspace, size_t workspace_bytes,
                                  void* stream);

/* As mxfp4_moe_decode_layer_routed with the step's post-attention residual,
 * RMSNorm and router projection in the same launch: the reference's
 *   x = x + o.bfloat16(); h2 = rms_norm(x) * w; logits = router(h2)
 *   (runtime/model_runner_v2.py:185-189, RMSNorm runtime/model_runner.py:20-25,
 *   the router through prequant + lin_pq on the MXFP4 rows of h2)
 * followed by the MoE of h2.  n_experts / 16 router workgroups compute the
 * logits and hand them to the launch's other workgroups (bounded wait, as
 * for h); the MoE runs on the un-quantized h2, as mxfp4_moe_decode_layer.
 * It has no single counterpart in the reference, whose step runs these as
 * separate launches (rmsnorm_lin_pq's pair of ops and the MoE); it saves a
 * launch per layer.  x bf16 (H), resid fp32 (H), norm_w bf16 (H); H = 2048;
 * router_wp / router_ws the MXFP4 router (n_experts, H/2) + (n_experts,
 * H/32), n_experts a multiple of 16 up to 256; optional outputs x_out (bf16
 * x + bf16(resid), the residual stream), y_out (bf16 h2), logits_out (fp32
 * logits), ids_out / w_out (both or neither).  Same workspace as
 * mxfp4_moe_decode_layer (launches of all three entry points may share one).
 */
int mxfp4_moe_decode_layer_fused_router(const void* x, const float* resid, const void* norm_w, float eps,
                                        const uint8_t* router_wp, const uint8_t* router_ws, int norm,
                                        void* x_out, void* y_out, float* logits_out, int32_t* ids_out,
                                        float* w_out, const uint8_t* gate_wp, const uint8_t* gate_ws,
                                        const uint8_t* up_wp, const uint8_t* up_ws, const uint8_t* down_wp,
                                        const uint8_t* down_ws, int n_experts, int E, int H, int Mi,
                                        float* out, void* workspace, size_t workspace_bytes, void* stream);

/* As mxfp4_moe_decode_layer_fused_router with the NEXT layer's input
 * residual, RMSNorm and q|k|v projection in the same launch, after the MoE:
 *   x_next = x_out + out.bfloat16(); qkv = lin_pq(MXFP4(rms_norm(x_next) * w))
 *   (runtime/model_runner_v2.py:208 then :147-152 of the next layer; the
 *   arithmetic of mxfp4_rmsnorm_lin_pq, whose outputs these equal bit for bit
 *   for Nq from 4081 to 8192, where that call also splits K in four)
 * ceil(Nq / 64) workgroups load the q|k|v rows while the MoE runs and wait
 * (bounded) for its output columns.  No single counterpart in the reference
 * (separate launches there); it saves the step another launch per layer.
 * qkv_norm_w bf16 (H); qkv_wp / qkv_ws the MXFP4 (Nq, H/2) + (Nq, H/32)
 * projection, Nq <= 8192; qkv_out fp32 (Nq); x_next_out optional bf16 (H),
 * which must not alias x or x_out.  16-byte aligned.  Same workspace as
 * mxfp4_moe_decode_layer.
 */
int mxfp4_moe_decode_layer_fused_router_qkv(const void* x, const float* resid, const void* norm_w, float eps,
                                            const uint8_t* router_wp, const uint8_t* router_ws, int norm,
                                            void* x_out, void* y_out, float* logits_out, int32_t* ids_out,
                                            float* w_out, const uint8_t* gate_wp, const uint8_t* gate_ws,
                                            const uint8_t* up_wp, const uint8_t* up_ws, const uint8_t* down_wp,
                                            const uint8_t* down_ws, int n_experts, int E, int H, int Mi,
                                            const void* qkv_norm_w, const uint8_t* qkv_wp, const uint8_t* qkv_ws,
                                            int Nq, float* qkv_out, void* x_next_out, float* out,
                                            void* workspace, size_t workspace_bytes, void* stream);

/* Everything of a decode layer after the attention scores, for one token
 * (batch 1), in one launch: the merge of the attention chunk records
 * (mxfp4_attn_decode_fused_partials' workspace; attn_decode's merge,
 * src/ext/mxfp4_decode.cu:366-430), o_proj on the MXFP4 of bf16(o)
 * (runtime/model_runner_v2.py:175-178, lin_pq), then
 * mxfp4_moe_decode_layer_fused_router_qkv (residual, RMSNorm, router, MoE and,
 * when qkv_wp is given, the next layer's input norm + q|k|v).  32 merge
 * workgroups and H/16 o_proj workgroups hand their rows on as tagged words
 * (bounded waits, as for h).  No single counterpart in the reference, whose
 * step runs these as separate launches; it leaves the step two launches per
 * layer.  The attention output (aq_out / as_out, optional) and oproj_out
 * equal attn_decode_mx's MXFP4 rows and lin_pq's output bit for bit.
 *   attn_workspace  the records of mxfp4_attn_decode_fused_partials (M = 1),
 *                   attn_workspace_bytes >= mxfp4_attn_decode_workspace_size(1,
 *                   Hq, max_pos); dpos the token's position (device)
 *   Hq = 32 query heads of 128 (o_proj K = 4096); o_wp / o_ws the MXFP4
 *   o_proj (H, 2048) + (H, 128); oproj_out fp32 (H), required
 *   x, norm_w, ... out, workspace: as mxfp4_moe_decode_layer_fused_router
 *   with resid = this launch's o_proj output; qkv_*: as
 *   mxfp4_moe_decode_layer_fused_router_qkv, or qkv_wp NULL for no tail.
 *   next_attn_workspace (with the tail; NULL for none): the NEXT layer's
 *   attention chunk pass also runs in this launch, as
 *   mxfp4_attn_decode_fused_partials(qkv_out, q_norm_next, k_norm_next, eps,
 *   theta, kvk_next, kvv_next, dpos, M = 1, Hq, Hkv, 128, max_pos, codec,
 *   next_attn_workspace) would: it writes the next layer's KV rows and
 *   chunk records for the next launch's merge, so a decode step is one
 *   launch per layer.  Hq = 8 Hkv, Nq = (Hq + 2 Hkv) * 128, max_pos * Hkv
 *   <= 32768; next_attn_workspace must differ from attn_workspace.
 * 16-byte aligned (aq_out 4-byte).  A position outside [0, max_pos) gives a
 * zero attention output.  Same workspace as mxfp4_moe_decode_layer.
 */
int mxfp4_decode_layer_post_attn(const void* attn_workspace, size_t attn_workspace_bytes, const int32_t* dpos,
                                 int Hq, int max_pos, uint8_t* aq_out, uint8_t* as_out, const uint8_t* o_wp,
                                 const uint8_t* o_ws, float* oproj_out, const void* x, const void* norm_w,
                                 float eps, const uint8_t* router_wp, const uint8_t* router_ws, int norm,
                                 void* x_out, void* y_out, float* logits_out, int32_t* ids_out, float* w_out,
                                 const uint8_t* gate_wp, const uint8_t* gate_ws, const uint8_t* up_wp,
                                 const uint8_t* up_ws, const uint8_t* down_wp, const uint8_t* down_ws,
                                 int n_experts, int E, int H, int Mi, const void* qkv_norm_w,
                                 const uint8_t* qkv_wp, const uint8_t* qkv_ws, int Nq, float* qkv_out,
                                 void* x_next_out, void* next_attn_workspace, size_t next_attn_workspace_bytes,
                                 uint8_t* kvk_next, uint8_t* kvv_next, const void* q_norm_next,
                                 const void* k_norm_next, int Hkv, float theta, int codec, float* out,
                                 void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------
 * A run of consecutive decode MoE layers in one launch (batch 1).  No single
 * reference entry point: it replaces the per-layer loop of
 * runtime/model_runner_v2.py:185-208 (prequant -> moe_gateup -> moe_down ->
 * moe_combine -> x + moe.bfloat16(), kernels src/ext/mxfp4_decode.cu:24-50,
 * 177-299) over layers 0..n_layers-1 when every layer's routing is known
 * before the launch, as in a stack of MoE layers with pre-drawn router
 * logits.  For each layer l, with e = ids[l][s]:
 *   y_l = sum_s w[l][s] * down_e(silu(gate_e x_l) * up_e x_l)  (fp32, as
 *   mxfp4_moe_decode_layer computes it), x_{l+1} = bf16(x_l + bf16(y_l)).
 *   x            bf16 (H) input of layer 0, 16-byte aligned
 *   ids, w       int32 / fp32 (n_layers, E) device arrays
 *   layer_table  device array of n_layers records of six pointers
 *                {gate_wp, up_wp, down_wp, gate_ws, up_ws, down_ws}, each
 *                the layer's experts stacked as for mxfp4_moe_decode_layer
 *   x_out        bf16 (H): x_{n_layers}
 *   x_all, y_all optional bf16 / fp32 (n_layers, H): x_{l+1} and y_l of
 *                every layer, or NULL
 *   strict       0: layer l+1's weights are fetched while layer l runs;
 *                1: a layer's weights are fetched only once its x is
 *                complete (the timing of routing that depends on x)
 *   workspace    mxfp4_decode_stack_workspace_size(E, H, Mi) bytes, 256-byte
 *                aligned, initialised once by mxfp4_decode_stack_reset; it
 *                needs no reset between launches or graph replays.
 * The launch's 256 workgroups run one per CU (slot s of the routing on XCD
 * s, the XCD's 32 CUs in two sets that compute alternate layers) and must
 * all be resident at once: the call fails with MXFP4_EINVAL unless the GPU
 * has 256 CUs (MI355X: 8 XCDs of 32), and no other kernel may occupy the GPU
 * meanwhile.  Every internal wait is bounded and an expired one is reported
 * by mxfp4_decode_stack_status.  Results are bit-identical to n_layers
 * chained mxfp4_moe_decode_layer launches.  Limits: E <= 8, H a multiple of
 * 512 up to 2048, Mi a multiple of 32 up to 1024.  The workspace holds a
 * 2 KB header and two buffers of 8-byte words, 8 * (2*Mi + 2*H) each (sizes
 * rounded up to 32 words).
 */
size_t mxfp4_decode_stack_workspace_size(int E, int H, int Mi);
int mxfp4_decode_stack_reset(void* workspace, int E, int H, int Mi, void* stream);
int mxfp4_decode_stack_status(const void* workspace, int* error_flag);
int mxfp4_moe_decode_stack(const void* x, const int32_t* ids, const float* w, const void* layer_table,
                           int n_layers, int n_experts, int E, int H, int Mi, void* x_out, void* x_all,
                           float* y_all, int strict, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------
 * The non-MoE ops of a decode step (the ops the reference's forward_decode / forward_batch run around the MoE,
 * runtime/model_runner_v2.py:130-300, so a whole step runs on this library).
 *
 * mxfp4_embed_rows: out (M, K) bf16 = the MXFP4 rows ids[m] (int32, device)
 * of an embedding (V, Kp/2) + (V, Kp/32), dequantized exactly:
 * bf16(sign * E2M1 * 2^(code-127)).  Replaces dequant_rows_gpu
 * (runtime/weight_store.py:47-65).  K a multiple of 8, out 16-byte aligned.
 */
int mxfp4_embed_rows(const uint8_t* wp, const uint8_t* ws, int V, int K, const int32_t* ids, int M,
                     void* out, void* stream);

/* mxfp4_rmsnorm_quant: per row m of x (M, H) bf16, optionally first
 * x_out = bf16(x + bf16(resid)) (resid fp32 (M, H), the residual add of
 * runtime/model_runner_v2.py:185/208), then y = rms_norm(x, w, eps) as
 * runtime/model_runner.py:20-25 computes it (fp32 mean of squares, bf16 of
 * x * rsqrt, times the bf16 weight, bf16) and its MXFP4 quantization yq
 * (M, H/2) / ys (M, H/32), bit-exact to mxfp4_prequant(y).  H a multiple of
 * 2048 up to 8192; pointers 16-byte aligned. */
int mxfp4_rmsnorm_quant(const void* x, const float* resid, const void* w, float eps, int M, int H,
                        void* x_out, void* y, uint8_t* yq, uint8_t* ys, void* stream);

/* mxfp4_rmsnorm_lin_pq: mxfp4_rmsnorm_quant followed by mxfp4_lin_pq on its
 * MXFP4 rows, in one launch: out (M, N) fp32 = MXFP4(rms_norm(x [+ resid]))
 * . W^T for W packed (N, H/2) + (N, H/32) -- the decode step's input norm +
 * q|k|v projection and post-attention norm + router
 * (runtime/model_runner_v2.py:147-152, :185-187; RMSNorm
 * runtime/model_runner.py:20-25).  No counterpart in the reference, which
 * launches the two separately.  x_out, y, yq/ys are the rmsnorm_quant outputs
 * and may each be NULL (x_out needs resid).  All outputs are bit-identical to
 * the two separate calls.  H = 2048, 1 <= M <= 16; x, resid, norm_w, x_out,
 * y, wp 16-byte aligned. */
int mxfp4_rmsnorm_lin_pq(const void* x, const float* resid, const void* norm_w, float eps, int M, int H,
                         void* x_out, void* y, uint8_t* yq, uint8_t* ys, const uint8_t* wp, const uint8_t* wsc,
                         int N, float* out, void* stream);

/* mxfp4_qk_norm_rope_kv: qkv fp32 (M, (Hq + 2 Hkv) * D) holds each token's q,
 * k and v projections side by side.  For token m at position *dpos + m:
 * q and k heads get RMSNorm with q_norm_w / k_norm_w (bf16 (D)) and the
 * half-layout RoPE of runtime/model_runner.py:28-41 (theta), q goes to
 * q_out (M, Hq, D) bf16, k and bf16(v) to the KV cache rows (max_pos, Hkv,
 * D) as E4M3 bytes.  codec 0: the decode extension's kv_write codec (as
 * mxfp4_kv_write; the graph runner's write, runtime/model_runner_v3.py:
 * 98-101); codec 1: torch's float8_e4m3fn conversion (round to nearest
 * even, 0x7F above 464; the batch step's write,
 * runtime/model_runner_v2.py:256-257).  D = 128. */
int mxfp4_qk_norm_rope_kv(const float* qkv, const void* q_norm_w, const void* k_norm_w, float eps,
                          float theta, const int32_t* dpos, int M, int Hq, int Hkv, int D, void* q_out,
                          uint8_t* kvk, uint8_t* kvv, int max_pos, int codec, void* stream);

/* mxfp4_argmax_advance: ids[m] = the first index of the maximum of logits
 * row m (M, V) fp32, NaN never winning -- greedy decoding,
 * runtime/decode_v2.py:71 -- and, when dpos is not NULL, *dpos += M once
 * every row is done.  ws: mxfp4_argmax_workspace_size(M, V) bytes, 256-byte
 * aligned, zero-filled once before its first use; every call leaves it
 * zero-filled again (so no clearing between calls or graph replays).  Calls
 * that share a workspace must not run concurrently. */
size_t mxfp4_argmax_workspace_size(int M, int V);
int mxfp4_argmax_advance(const float* logits, int M, int V, int32_t* ids, int32_t* dpos, void* ws,
                         size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------------
 * Token -> expert grouping (the bookkeeping of torch.where(topi == e) in
 * runtime/model_runner_v2.py:111 and of the token-major tables :279-286).
 * topi int64 (T, topk) device ids.  Writes counts[e] (pairs routed to e),
 * offsets[e] (number of valid pairs with a smaller id) and pairs[offsets[e]
 * + i] = t*topk + k for the i-th such pair in row-major order -- a stable sort
 * of the pairs by expert id.  Ids outside [0, n_experts) are left out.
 * counts/offsets hold n_experts ints, pairs T*topk ints; n_experts <= 1024.
 */
int mxfp4_moe_group(const int64_t* topi, int T, int topk, int n_experts, int* counts, int* offsets,
                    int* pairs, void* stream);

/* ---------------------------------------------------------------------
 * Router top-k on the GPU.  Replaces the host-side routing of every MoE
 * layer (runtime/model_runner_v2.py:189-192 decode, :272-275 batch, and
 * moe_route :100-105):  probs = softmax(logits.float(), -1);
 * topv, topi = topk(probs, k); topv /= topv.sum(-1) if norm.
 *   logits  fp32 (M, n_experts), rows ldl floats apart
 *   ids     int32 (M, k) out, descending probability (exact ties: lower
 *           index first; torch.topk leaves their order unspecified)
 *   ids64   optional int64 (M, k) out (torch's topi layout), or NULL
 *   w       fp32 (M, k) out: topv, renormalised over the k winners (summed
 *           in rank order) when norm != 0
 * n_experts <= 1024, k <= min(32, n_experts).  The ids feed the fused layer's
 * device routing (mxfp4_moe_decode_layer ids_dev/w_dev) or
 * mxfp4_route_tables, with no host round trip.
 */
int mxfp4_route_topk(const float* logits, int64_t ldl, int M, int n_experts, int k, int norm,
                     int32_t* ids, int64_t* ids64, float* w, void* stream);

/* ---------------------------------------------------------------------
 * Device pointer tables of the drop-in grouped ops from device ids: the
 * token-major lists the reference builds on the host and copies to the
 * device (runtime/model_runner_v2.py:279-286, src/ext/mxfp4_decode_binding.cpp:
 * 44-60).  For row m, slot e (ids int32 (M, k)):
 *   gu_wp_tab[m*2k + e]     = gate_wp + id*Mi*Kp_h/2,  [m*2k + k + e] = up
 *   gu_ws_tab[...]          the same for the scales (Mi*Kp_h/32 per expert)
 *   dn_wp_tab[m*k + e]      = down_wp + id*H*Kp_mi/2,  dn_ws_tab likewise
 * over weights stacked per layer as for mxfp4_moe_decode_layer (Kp_h, Kp_mi
 * = H, Mi rounded up to 32).  The tables are what mxfp4_moe_gateup_devtab /
 * mxfp4_moe_down_devtab take.  Ids outside [0, n_experts) are clamped into
 * range (memory safety only; routing produced by mxfp4_route_topk is valid).
 */
int mxfp4_route_tables(const int32_t* ids, int M, int k, const uint8_t* gate_wp, const uint8_t* gate_ws,
                       const uint8_t* up_wp, const uint8_t* up_ws, const uint8_t* down_wp,
                       const uint8_t* down_ws, int n_experts, int H, int Mi, int64_t* gu_wp_tab,
                       int64_t* gu_ws_tab, int64_t* dn_wp_tab, int64_t* dn_ws_tab, void* stream);

/* ---------------------------------------------------------------------
 * The MoE block of a batched decode step (M <= 16 tokens), two launches.
 * Replaces the moe_gateup -> moe_down -> moe_combine chain of
 * ModelRunnerV2.forward_batch (runtime/model_runner_v2.py:265-289; kernels
 * src/ext/mxfp4_decode.cu:177-299) over weights stacked per layer as for
 * mxfp4_moe_decode_layer, with the same arithmetic: MXFP4 activation rows,
 * g and u in fp32, h = silu(g)*u quantized to MXFP4 per 32-block, down on
 * MXFP4 h, the weighted sum of a token's E slots in fp32.  Each routed
 * expert's weights are read once per call however many tokens share it.
 *   xq, xs   MXFP4 rows of the normed activations, (M, H/2) and (M, H/32)
 *            (mxfp4_prequant / mxfp4_rmsnorm_quant output), 16-byte aligned
 *   ids, w   int32 / fp32 (M, E) expert ids and routing weights
 *            (mxfp4_route_topk output); ids outside [0, n_experts)
 *            contribute nothing
 *   y        fp32 (M, H) MoE output, overwritten: the gate/up launch clears
 *            it and the down launch adds two partial sums per element with
 *            device-scope fp32 atomics (a fixed pair, so the result is
 *            deterministic).  y must be ordinary device memory (not host-
 *            mapped or fine-grained) and nothing may read or write it
 *            between the entry's two launches.
 *   ws       mxfp4_moe_decode_batch_workspace_size(M, E, Mi) bytes, 16-byte
 *            aligned (the per-slot MXFP4 h and the owner table the gate/up
 *            launch hands to the down launch; nothing persists)
 * Limits: 1 <= M <= 16, 1 <= E <= 8, H a multiple of 128, Mi of 32.  The
 * sums match the drop-in chain up to fp32 summation order.
 */
size_t mxfp4_moe_decode_batch_workspace_size(int M, int E, int Mi);
int mxfp4_moe_decode_batch(const uint8_t* xq, const uint8_t* xs, const int32_t* ids, const float* w,
                           const uint8_t* gate_wp, const uint8_t* gate_ws, const uint8_t* up_wp,
                           const uint8_t* up_ws, const uint8_t* down_wp, const uint8_t* down_ws, int n_experts,
                           int M, int E, int H, int Mi, float* y, void* ws, size_t ws_bytes, void* stream);

/* mxfp4_moe_decode_batch_noalloc: mxfp4_moe_decode_batch with its h staged
 * in a fixed scratch array of the library (141,568 bytes per GPU, held until
 * the process ends) instead of a caller workspace.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops).  It calls no allocator.  Limits as
 * mxfp4_moe_decode_batch plus Mi <= 2048; larger shapes return MXFP4_EINVAL.
 * Every call on one GPU shares that GPU's scratch: calls that overlap in time
 * on one GPU (different streams, no ordering) race and give wrong results;
 * stream-ordered calls are safe.  Nothing is kept between calls. */
int mxfp4_moe_decode_batch_noalloc(const uint8_t* xq, const uint8_t* xs, const int32_t* ids, const float* w,
                                   const uint8_t* gate_wp, const uint8_t* gate_ws, const uint8_t* up_wp,
                                   const uint8_t* up_ws, const uint8_t* down_wp, const uint8_t* down_ws,
                                   int n_experts, int M, int E, int H, int Mi, float* y, void* stream);

/* ---------------------------------------------------------------------
 * Grouped MoE over a batch of tokens (prefill, speculative verify).
 * Replaces ModelRunnerV2.moe_compute (runtime/model_runner_v2.py:108-122):
 * per expert e the rows of torch.where(topi == e) go through `forward` with
 * gate_e and up_e (activations rounded to fp16, then MXFP4), h = silu(g)*u in
 * fp32, `forward` with down_e (h rounded to fp16, then MXFP4), .to(bf16),
 * times the bf16 score, accumulated into a bf16 output.
 *   x        bf16 (T, H), 16-byte aligned
 *   topi     int64 (T, topk) expert ids; ids outside [0, n_experts)
 *            contribute nothing (as an id absent from the reference's
 *            `experts` dict)
 *   scores   bf16 (T, topk)
 *   weights  stacked per layer exactly as for mxfp4_moe_decode_layer
 *   out      bf16 (T, H), 16-byte aligned: the slots of a token are summed
 *            in fp32 in slot order and rounded once (the reference adds in
 *            bf16 in expert order)
 *   workspace >= mxfp4_moe_prefill_workspace_size(T, topk, n_experts, H, Mi)
 *            bytes, 256-byte aligned; no state is kept between calls.
 * Limits: H, Mi multiples of 32; 0 < topk <= 32; n_experts <= 1024.
 */
size_t mxfp4_moe_prefill_workspace_size(int T, int topk, int n_experts, int H, int Mi);
int mxfp4_moe_prefill(const void* x, const int64_t* topi, const uint16_t* scores,
                      const uint8_t* gate_wp, const uint8_t* gate_ws, const uint8_t* up_wp,
                      const uint8_t* up_ws, const uint8_t* down_wp, const uint8_t* down_ws,
                      int n_experts, int T, int topk, int H, int Mi, void* out, void* workspace,
                      size_t workspace_bytes, void* stream);

/* As mxfp4_moe_prefill with the experts given by a device table of
 * n_experts x 6 int64 pointers (gate wp, gate wsc, up wp, up wsc, down wp,
 * down wsc) -- the per-expert spec dicts of runtime/weight_store.py:278-284.
 * Every id that can occur must have non-null entries. */
int mxfp4_moe_prefill_tab(const void* x, const int64_t* topi, const uint16_t* scores,
                          const int64_t* expert_tab, int n_experts, int T, int topk, int H, int Mi,
                          void* out, void* workspace, size_t workspace_bytes, void* stream);

/* Test hook, no counterpart in the reference: for each of n_waves groups of
 * 64 floats, every lane's wave sum as the RMSNorm kernels reduce it
 * (permlane swaps + DPP, out_butterfly) and by the __shfl_xor butterfly
 * (out_xor), so the GPU tests can pin the two as bit-identical. */
int mxfp4_selftest_wave_sum(const float* in, float* out_butterfly, float* out_xor, int n_waves, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* MXFP4_HIP_H */
