/*
 * sluice_decoder.h - kernels of the synthetic decoders that carry the
 * routed-MoE decode path in the benchmarks (DeepSeek-V2-Lite-shaped MLA
 * attention, Qwen3-MoE-shaped GQA attention with q/k norm, RMSNorm with a
 * fused residual add, SwiGLU activation, router logits).  They are not part
 * of the reference's interface: the reference runs these layers inside
 * vLLM; here they replace chains of small torch ops so a decode step spends
 * its time in the MoE path rather than in kernel launches.
 *
 * Same conventions as sluice.h: int status (0 ok, positive hipError_t,
 * negative SLUICE_E_*), plain device pointers, asynchronous on `stream`.
 * Activations and weights are bf16 (uint16 storage); positions and step
 * counters are int64 device scalars/arrays (torch long).  Every kernel
 * checks a position against the cache length and skips rows outside it.
 */
#ifndef SLUICE_DECODER_H_
#define SLUICE_DECODER_H_

#include <stddef.h>
#include <stdint.h>

#include "sluice.h"

#ifdef __cplusplus
extern "C" {
#endif

/* x [rows, H] becomes bf16(x + delta) in place when delta != NULL; then
 * out [rows, H] = bf16(x * rsqrt(mean(x^2) + eps) * w), fp32 arithmetic.
 * H % 8 == 0. */
int sluice_dec_add_rmsnorm(void* x, const void* delta, const void* w, void* out, int rows, int H,
                           float eps, sluice_stream_t stream);

/* Skinny GEMM: y [T, N] = bf16(x [T, K] . w [N, K]^T), fp32 accumulation,
 * T <= 16, N % 16 == 0, K % 64 == 0 (weights streamed once on MFMA bf16).
 * workspace (16-byte aligned, sluice_dec_linear_workspace() bytes,
 * zero-filled before its first use; every call leaves it so) lets a small
 * matrix split K over more workgroups; NULL runs without the split.  Calls
 * sharing a workspace must not overlap. */
size_t sluice_dec_linear_workspace(void);
int sluice_dec_linear(const void* x, const void* w, int T, int N, int K, void* y,
                      void* workspace, sluice_stream_t stream);

/* The plain projection left as its K parts: parts [ks, T, N] fp32 (row-major,
 * 16-byte aligned), ks = sluice_dec_linear_split_parts(T, N, K) (>= 1, 0 for
 * a shape it does not take).  bf16(sum of the parts in order) is the
 * projection; it can differ from what sluice_dec_linear writes by the fp32
 * rounding of a different K split (the two may split K differently). */
int sluice_dec_linear_split_parts(int T, int N, int K);
int sluice_dec_linear_split(const void* x, const void* w, int T, int N, int K, float* parts,
                            sluice_stream_t stream);

/* Gate/up projection with the SwiGLU activation applied to its fp32 sums:
 * w [N, K] holds N/2 gate rows then N/2 up rows; y [T, N/2] =
 * bf16(silu(x . w_gate^T) * (x . w_up^T)).  N % 32 == 0; workspace as for
 * sluice_dec_linear. */
int sluice_dec_linear_glu(const void* x, const void* w, int T, int N, int K, void* y,
                          void* workspace, sluice_stream_t stream);

/* Greedy next token: out[t] (int64) = the first index of the largest value
 * of x [T, N] bf16 (NaN never wins; an all-NaN row gives 0).  One launch
 * with no memset, so it is safe inside a replayed hipGraph. */
int sluice_dec_argmax(const void* x, int T, int N, int64_t* out, sluice_stream_t stream);

/* out [rows, I] = bf16(silu(gu[:, :I]) * gu[:, I:]), gu [rows, 2I].  I % 4 == 0. */
int sluice_dec_silu_mul(const void* gu, void* out, int rows, int I, sluice_stream_t stream);

/* Router logits: out [rows, E] fp32 = hn [rows, H] . wg [E, H]^T, plus
 * bias_table[(step % n_steps) * bias_rows + t][e] when bias_table != NULL
 * (step read from device memory).  rows <= 16, H % 512 == 0. */
int sluice_dec_gate_logits(const void* hn, const void* wg, const float* bias_table,
                           const int64_t* step, int n_steps, int bias_rows, int rows, int H, int E,
                           float* out, sluice_stream_t stream);

/* Residual add + RMSNorm + router logits in one launch:
 *   x_out = bf16(x + delta) (x when delta is NULL), hn_out = bf16(rmsnorm(x_out) * w)
 *   (bit-identical to sluice_dec_add_rmsnorm), logits as sluice_dec_gate_logits
 *   computes them from hn_out (bit-identical when H == 2048).  The delta may
 *   instead come as delta_parts [n_parts, rows, H] fp32 (n_parts <= 4, delta
 *   NULL): delta = bf16(sum of the parts in order), as sluice_dec_linear_split
 *   leaves a projection.  x_out must not
 *   alias x.  Shapes it takes: sluice_dec_add_rmsnorm_gate_ok(rows, H) != 0
 *   (H % 8 == 0, H <= 8192, rows <= 16); pointers 16-byte aligned. */
int sluice_dec_add_rmsnorm_gate_ok(int rows, int H);
int sluice_dec_add_rmsnorm_gate(const void* x, const void* delta, const float* delta_parts,
                                int n_parts, const void* w, void* x_out, void* hn_out,
                                const void* wg, const float* bias_table,
                                const int64_t* step, int n_steps, int bias_rows, int rows, int H,
                                int E, float eps, float* logits, sluice_stream_t stream);

/* MLA decode (DeepSeek-V2 latent attention with absorbed up-projections) on
 * the matrix cores, three launches (q absorption + new cache rows, row splits
 * of the attention, merge + value up-projection):
 *   q rows of q_stride elements hold nh heads of (nope then rope) values,
 *   kva rows of kva_stride elements hold lora then rope values;
 *   q_lat = q_nope . w_uk[h] (w_ukt [nh, lora, nope] is w_uk transposed),
 *   q_pe = rope(q_pe); ckv_cache [c, L, lora] row pos[t] =
 *   bf16(rmsnorm(kva[:lora]) * kv_norm), kpe_cache [c, L, rope] row pos[t] =
 *   bf16(rope(kva[lora:])); scores over cache rows 0..pos[t] =
 *   (q_lat . ckv + q_pe . kpe) * scale, softmax, o_lat = p . ckv,
 *   out [c, nh*vh] = bf16(o_lat . w_uv[h]) (w_uv [nh, lora, vh]).
 * rope is rotate-half with cos/sin [*, rope/2] fp32 rows at pos[t].  The
 * latent cache is kept twice: ckv_cache and ckvt_cache [c, L/32, lora, 32],
 * row r of each 32-row block at slot 8*((r & 15) >> 2) + 4*(r >> 4) + (r & 3)
 * of each latent column; row pos[t] is written to both.  q_lat and p are
 * rounded to bf16 for the products.  lora == 512, rope == 64, nh % 16 == 0,
 * nope % 32 == 0, vh % 8 == 0 and <= 256, c <= 16, L % 32 == 0 and <= 4096.
 * work: sluice_dec_mla_workspace(c, nh) bytes; q, w_ukt, w_uv, the caches and
 * work 16-byte aligned, kva and kv_norm 4-byte aligned. */
size_t sluice_dec_mla_workspace(int c, int nh);
int sluice_dec_mla_decode(const void* q, int q_stride, const void* kva, int kva_stride,
                          const void* kv_norm, const void* w_ukt, const void* w_uv,
                          const float* cos_t, const float* sin_t, const int64_t* pos, int c,
                          int nh, int nope, int rope, int lora, int vh, int L, float eps,
                          float scale, void* ckv_cache, void* ckvt_cache, void* kpe_cache,
                          void* work, void* out, sluice_stream_t stream);

/* GQA decode with per-head q/k RMSNorm (Qwen3-MoE), one launch:
 *   from qkv [c, (nh + 2*kvh)*hd]: q_h = rope(rmsnorm(q_h) * q_norm) (bf16),
 *   k_cache [c, kvh, L, hd] row pos[t] = bf16(rope(rmsnorm(k_g) * k_norm)),
 *   v_cache [c, kvh, L, hd] row pos[t] = v_g; then per query head h (kv head
 *   h / (nh/kvh)): softmax over rows 0..pos[t] of (q . k) * scale,
 *   out [c, nh*hd] = bf16(p . v).  hd == 128, L <= 4096; qkv, q_norm,
 *   k_norm, cos_t, sin_t and the caches 16-byte aligned, out 4-byte aligned.
 *   Exactly one of qkv and qkv_parts: the QKV projection's K parts
 *   [n_parts, c, (nh + 2*kvh)*hd] fp32 (n_parts <= 4, as sluice_dec_linear_split
 *   leaves them) are summed in order and rounded to bf16 first. */
int sluice_dec_gqa_decode(const void* qkv, const float* qkv_parts, int n_parts,
                          const void* q_norm, const void* k_norm,
                          const float* cos_t, const float* sin_t, const int64_t* pos, int c,
                          int nh, int kvh, int hd, int L, float eps, float scale, void* k_cache,
                          void* v_cache, void* out, sluice_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SLUICE_DECODER_H_ */
