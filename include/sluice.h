/*
 * sluice.h - C ABI of libsluice_hip.so, the MI355X (gfx950) routed-MoE decode
 * hot path of Sluice: top-k routing, the streaming gap (slot-cache hit/miss,
 * expert H2D copies, expert-map refresh), the grouped SwiGLU expert product
 * over slot buffers and the weighted combine.
 *
 * Conventions
 *   - Every entry point returns int: 0 on success, a positive hipError_t from
 *     the HIP runtime, or a negative SLUICE_E_* code.  Nothing throws across
 *     the ABI.  sluice_strerror() turns a code into text.
 *   - Device pointers are plain device addresses (torch data_ptr()), host
 *     pointers are host addresses; no torch types appear in any signature.
 *   - Work is enqueued on the hipStream_t the caller passes (torch's
 *     current_stream().cuda_stream); calls are asynchronous unless stated.
 *   - Integer ids are int32, routing weights fp32, activations and unquantized
 *     weights bf16 (uint16 storage), fp8 weights OCP e4m3fn (uint8 storage).
 *
 * Each declaration names the reference interface it replaces
 * (kfirtoledo/sluice file:line, vLLM 0.23 call sites).
 */
#ifndef SLUICE_H_
#define SLUICE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* sluice_stream_t; /* == hipStream_t */

#define SLUICE_OK 0
#define SLUICE_E_INVAL (-1)    /* bad argument / shape outside kernel limits */
#define SLUICE_E_OVERFLOW (-2) /* working set exceeds slots (reference raises) */
#define SLUICE_E_TIMEOUT (-3)  /* a bounded gap wait (host or device) timed out */
#define SLUICE_E_NOMEM (-4)    /* host allocation failed */
#define SLUICE_E_STATE (-5)    /* object used in a state it does not allow */
#define SLUICE_E_ABORTED (-6)  /* a device gap wait ended by the abort flag */
#define SLUICE_E_SCRATCH (-7)  /* call too large for the no-alloc entry's scratch */
#define SLUICE_E_COPY (-8)     /* a host-to-device row copy failed to issue or complete */

/* Kernel limits (checked on the host before every launch). */
#define SLUICE_MAX_EXPERTS 1024  /* global experts E per layer */
#define SLUICE_MAX_SLOTS 512     /* slots S per layer */
#define SLUICE_MAX_TOPK 16       /* k */
#define SLUICE_MAX_PAIRS 4096    /* T*k (token, expert) pairs per call */
#define SLUICE_BLOCK_M 16        /* tokens per aligned block */

#define SLUICE_ABI_VERSION 1

int sluice_abi_version(void);
const char* sluice_strerror(int code);

/* ------------------------------------------------------------------------
 * a1. Top-k routing.  Replaces vLLM's runner.router.select_experts
 * (called at src/sluice/offloader.py:2583-2585).  One wave64 per token.
 *   scoring 0 = softmax: select on logits (softmax is monotone), ties go to
 *               the lower expert id; weight = softmax prob (fp32);
 *   scoring 1 = sigmoid: s = fp32(1/(1+exp(-x))) evaluated in fp64 and
 *               rounded once; selection on fp32(s + bias); weight = s.
 *   n_group > 1 enables group-limited selection: group score is the max
 *   logit (softmax) or the sum of the two largest biased scores (sigmoid);
 *   only the topk_group best groups (ties: lower group id) stay eligible.
 *   renorm divides the k weights by their sum (+1e-20 for sigmoid), then
 *   every weight is multiplied by scale.
 * logits [T,E] (dtype 0 = fp32, 1 = bf16), bias [E] fp32 or NULL,
 * ids_out [T,k] int32, w_out [T,k] fp32, both in descending score order.
 * ---------------------------------------------------------------------- */
int sluice_route_topk(const void* logits, int logits_dtype, int T, int E, int k,
                      int scoring, int renorm, float scale, const float* bias,
                      int n_group, int topk_group, int32_t* ids_out,
                      float* w_out, sluice_stream_t stream);

/* ------------------------------------------------------------------------
 * a4. Slot lookup.  Replaces the gap's ids D2H + sorted(set(ids)) + residency
 * scan (src/sluice/offloader.py:2406-2441).  One workgroup builds an LDS
 * presence map over the E experts, compacts the selected ids in ascending
 * order with wave ballots, counts owned-but-unmapped ids (misses against a
 * standing map) and publishes the record to `rec` (host-mapped pinned memory
 * or device memory), writing rec->stamp = stamp last with a system-scope
 * release store.
 * ---------------------------------------------------------------------- */
typedef struct sluice_gap_record {
  volatile int32_t stamp;
  int32_t n_uniq;
  int32_t n_miss;
  int32_t reserved;
  int32_t uniq[SLUICE_MAX_EXPERTS];
} sluice_gap_record;

int sluice_slot_lookup(const int32_t* ids, int n, const int32_t* expert_map,
                       const int32_t* local_of, int E, sluice_gap_record* rec,
                       int32_t stamp, sluice_stream_t stream);

/* ------------------------------------------------------------------------
 * a7. Standing expert-map refresh.  Replaces _write_map/_write_standing_map
 * (src/sluice/offloader.py:2083-2123): map = -1 everywhere, then
 * map[slot_global[s]] = s for every occupied slot s (slot_global[s] < 0 =
 * empty).  The S-entry table travels as a kernel argument, so no pinned
 * staging buffer and no host wait on a previous copy are needed.
 * slot_global is a HOST array; map is device [E] int32.
 * ---------------------------------------------------------------------- */
int sluice_map_refresh(int32_t* expert_map, int E, const int32_t* slot_global,
                       int S, sluice_stream_t stream);

/* ------------------------------------------------------------------------
 * a6. Expert H2D streaming.  Replaces _stream_in (src/sluice/offloader.py:
 * 2709-2723): n row copies dst[i] <- src[i] of bytes[i] each, issued as
 * hipMemcpyAsync on `stream` (the caller's dedicated copy stream).
 * ---------------------------------------------------------------------- */
int sluice_copy_rows(void* const* dst, const void* const* src,
                     const size_t* bytes, int n, sluice_stream_t stream);

/* Pinned host store for the experts (replaces `cpu.pin_memory()` in
 * _install_cache, src/sluice/offloader.py:965-967): hipHostMalloc of exactly
 * `bytes` (no power-of-two rounding), portable across devices. */
int sluice_host_alloc(size_t bytes, void** out);
int sluice_host_free(void* p);

/* ------------------------------------------------------------------------
 * a9/a10. Grouped SwiGLU expert product over slot buffers + weighted combine.
 * Replaces torch.ops.vllm.fused_experts(h, w13, w2, tw, ti, activation=
 * "silu", global_num_experts=E, expert_map=map) (src/sluice/offloader.py:
 * 2590-2599) and vLLM's moe_sum.
 *   x [T,H] bf16; w13 [S,2I,H] (gate rows, then up rows); w2 [S,H,I];
 *   topk_w [T,k] fp32; topk_ids [T,k] int32 global ids; expert_map [E]
 *   int32 (global -> slot, -1 = not resident: the pair contributes 0) or
 *   NULL (identity, ids are slots);
 *   out[t] = bf16( scale * sum_j w[t,j] * W2[s]·(silu(W13g[s]·x_t) * W13u[s]·x_t)
 *                  + SharedMLP(x_t) + shared[t] )
 *   shared (may be NULL): a precomputed shared-expert output [T,H] bf16.
 *   SharedMLP: the layer's shared experts run inside the same grouped
 *     product (the traced tail's shared_experts(x), offloader.py:341-342,
 *     2602, added unscaled): shared_w13 [2*shared_I, H] (gate rows, then up
 *     rows), shared_w2 [H, shared_I]; shared_I a multiple of I (at most
 *     4*I), or 0 with NULL weights for none.  It is computed as shared_I/I
 *     groups of I channels, each one more expert block over every token.
 * fp8 variant: w13/w2 are e4m3fn with fp32 block scales of block_n x block_k
 * (128x128): w13_scale [S, ceil(2I/bn), ceil(H/bk)], w2_scale
 * [S, ceil(H/bn), ceil(I/bk)]; activations stay bf16.  Shared weights are
 * e4m3fn too, with shared_w13_scale [2*shared_I/128, H/128] and
 * shared_w2_scale [H/128, shared_I/128].
 * Requires H % 64 == 0, I % 64 == 0, E <= SLUICE_MAX_EXPERTS,
 * T*(k + shared_I/I) <= SLUICE_MAX_PAIRS.
 * The workspace (device) must hold sluice_fused_experts_workspace() bytes;
 * it needs no initial contents and keeps none between calls (calls that
 * share one must not overlap).
 * plan (may be NULL): the plan of these topk_ids over this expert_map (the
 * sluice_moe_align layout), built on `stream` before the call -- by the
 * layer's gap (sluice_layer_gap_launch with a plan buffer), which leaves the
 * map this call reads; the call then launches no align kernel of its own.
 * NULL: the call builds the plan in its workspace.
 * ---------------------------------------------------------------------- */
size_t sluice_fused_experts_workspace(int T, int H, int I, int k, int shared_I);

int sluice_fused_experts_bf16(const void* x, const void* w13, const void* w2,
                              const float* topk_w, const int32_t* topk_ids,
                              const int32_t* expert_map, int T, int H, int I,
                              int k, int E, int S, float scale,
                              const void* shared_w13, const void* shared_w2,
                              int shared_I, const void* shared, void* workspace,
                              size_t workspace_bytes, void* out, const int32_t* plan,
                              sluice_stream_t stream);

/* No-allocation variant of sluice_fused_experts_bf16 (same arguments minus
 * the workspace, same kernels, bit-identical results).  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * hipGraph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Its scratch is a fixed device array of SLUICE_NOALLOC_SCRATCH_BYTES in the
 * library, one per GPU, held until the process ends; the call allocates and
 * frees nothing.  Calls needing more than that
 * (sluice_fused_experts_workspace(T, H, I, k, shared_I) bytes) return
 * SLUICE_E_SCRATCH before any device work.  The scratch needs no initial
 * contents; every call on a GPU shares that GPU's copy, so calls that overlap
 * on one GPU (different streams or threads) race and must be serialised by
 * the caller.  The current device must be the one x, the weights and stream
 * belong to.  The first call on a device looks the scratch's address up. */
#define SLUICE_NOALLOC_SCRATCH_BYTES (8u << 20)
int sluice_fused_experts_bf16_noalloc(const void* x, const void* w13, const void* w2,
                                      const float* topk_w, const int32_t* topk_ids,
                                      const int32_t* expert_map, int T, int H, int I,
                                      int k, int E, int S, float scale,
                                      const void* shared_w13, const void* shared_w2,
                                      int shared_I, const void* shared, void* out,
                                      const int32_t* plan, sluice_stream_t stream);

int sluice_fused_experts_fp8(const void* x, const void* w13,
                             const float* w13_scale, const void* w2,
                             const float* w2_scale, int block_n, int block_k,
                             const float* topk_w, const int32_t* topk_ids,
                             const int32_t* expert_map, int T, int H, int I,
                             int k, int E, int S, float scale,
                             const void* shared_w13, const float* shared_w13_scale,
                             const void* shared_w2, const float* shared_w2_scale,
                             int shared_I, const void* shared, void* workspace,
                             size_t workspace_bytes, void* out, const int32_t* plan,
                             sluice_stream_t stream);

/* Token permute / align-to-block (vLLM moe_align_block_size): groups the
 * T*k (token, expert) pairs by slot into blocks of <= SLUICE_BLOCK_M pairs,
 * slots ascending, pairs ascending within a slot.  plan (device int32):
 *   plan[0] = n_blocks, plan[1] = T*k, plan[2] = n_resident; then per block
 *   18 ints {slot field, count, pair[16]} starting at plan[4]; then T*k
 *   validity flags at plan[4 + 18*T*k].  Slots whose rows a router-split gap
 *   of this map is still streaming come last, their slot field or-ed with
 *   1<<30; the n_resident blocks before them are the others.  The shared
 *   experts' blocks are not in the plan (the product derives them).  Exposed
 *   for testing; fused_experts runs it itself unless given a plan. */
size_t sluice_moe_plan_ints(int T, int k);
int sluice_moe_align(const int32_t* topk_ids, int T, int k,
                     const int32_t* expert_map, int E, int S, int32_t* plan,
                     sluice_stream_t stream);

/* The three compute stages of sluice_fused_experts_bf16 (and the fp8 gemms
 * of sluice_fused_experts_fp8, with the same block-scale layout), launchable one by
 * one over a plan from sluice_moe_align (for per-kernel timing and tests):
 *   gemm1:   act[pair, I] (bf16) = silu(W13g[s]·x_t) * W13u[s]·x_t
 *   gemm2:   partial[pair, H] (fp32) = w[pair] * W2[s]·act[pair]
 *   combine: out[t] = bf16(scale * sum_j valid ? partial[t*k+j] : 0 + shared)
 * Shapes and alignment as for sluice_fused_experts_bf16. */
int sluice_moe_gemm1_bf16(const void* x, const void* w13, const int32_t* plan,
                          int T, int H, int I, int k, void* act,
                          sluice_stream_t stream);
int sluice_moe_gemm2_bf16(const void* act, const void* w2,
                          const int32_t* plan, const float* topk_w, int T,
                          int H, int I, int k, float* partial,
                          sluice_stream_t stream);
int sluice_moe_gemm1_fp8(const void* x, const void* w13, const float* w13_scale,
                         const int32_t* plan, int T, int H, int I, int k, void* act,
                         sluice_stream_t stream);
int sluice_moe_gemm2_fp8(const void* act, const void* w2, const float* w2_scale,
                         const int32_t* plan, const float* topk_w, int T, int H, int I,
                         int k, float* partial, sluice_stream_t stream);
int sluice_moe_combine(const float* partial, const int32_t* plan, int T, int k,
                       int H, float scale, const void* shared, void* out,
                       sluice_stream_t stream);

/* ------------------------------------------------------------------------
 * a2-a8. Per-layer slot cache + gap.  Replaces _ExpertLayerCache
 * (src/sluice/offloader.py:121-169), _install_cache's slot/map layout
 * (895-1044), the SLRU core _touch/_coldest_protected/_acquire_slot/
 * _evict_to (2009-2081) and _router_split_gap (2362-2467).  Slot
 * assignment follows the reference's OrderedDict semantics exactly.
 * ---------------------------------------------------------------------- */
typedef struct sluice_layer sluice_layer;

/* local_of [E] host array: global id -> local expert (or -1 = not owned).
 * expert_map_dev: the device map buffer (may be NULL for host-only use, in
 * which case sluice_layer_gap_host is the only gap entry allowed). */
int sluice_layer_create(int E, int local_n, int num_slots, int protected_cap,
                        const int32_t* local_of, int32_t* expert_map_dev,
                        sluice_layer** out);
int sluice_layer_destroy(sluice_layer* layer);

/* Register one per-expert parameter: slot buffer base (device, [S, row])
 * and pinned host store base ([local_n, row]), row_bytes per expert.  On a
 * layer with a device map both ranges must lie whole inside allocations the
 * HIP/HSA runtime made or locked (SLUICE_E_INVAL otherwise): the gap copies
 * rows with the SDMA engines directly.
 * On a layer with a device map, params with rows of at most 32 KB (whole
 * 16-byte vectors; up to 4 such params) are copied into HBM whole here
 * (local_n rows), and a gap answered before its rows land copies their rows
 * into the filled slots from there in the gap kernel, so such host rows must
 * hold their final contents when the param is registered.  A gap's other
 * rows go to the SDMA engines through the HSA runtime (two copy lanes); the
 * classic wave path copies with hipMemcpyAsync on HIP copy streams. */
int sluice_layer_add_param(sluice_layer* layer, void* slot_base_dev,
                           const void* host_base, size_t row_bytes);

/* No counterpart in the reference.  How many of the layer's params the gap
 * kernel copies itself (see sluice_layer_add_param). */
int sluice_layer_pulled_params(sluice_layer* layer);

/* No counterpart in the reference.  Staging rows: `rows` (0..8) experts per
 * layer kept in HBM outside the slots, each a copy of one expert the layer
 * selects often but does not hold (the most selected ones, by counts of
 * the gaps' selections halved every 4096 gaps).  A gap server fills them
 * from the host store while the host link idles, in 2 MiB chunks on two
 * SDMA engines the gap's own copies do not use, at most two chunks in
 * flight per server.  A gap answered before its rows land copies a miss
 * whose expert is staged into its slot from HBM with the runtime's
 * device-to-device copy (a copy kernel: ~29 us for a 17.3 MB expert
 * instead of ~310 us over the link), and answers the device once those
 * copies landed (no kernel then waits for a copy that needs CUs); the
 * misses that cross the link are queued meanwhile.  Slot assignment, maps
 * and slot bytes are what they are without staging.  Costs rows x (bytes of
 * the non-pulled params' rows) of HBM.  Call after every
 * sluice_layer_add_param (which then returns SLUICE_E_STATE) with no gap
 * server attached to the layer, not under graph capture (it allocates); a
 * call with the count already set changes nothing.  SLUICE_E_INVAL when the
 * runtime reports no SDMA engines free for the staging copies. */
int sluice_layer_set_staging(sluice_layer* layer, int rows);
/* counters[6]: rows, rows holding an expert whole, rows filled so far,
 * host-to-device bytes of staging copies, misses copied into their slots
 * from a staged row, and those misses' bytes. */
int sluice_layer_stage_counters(const sluice_layer* layer, int64_t* counters);

/* Coded host stores: no counterpart in the reference, which streams the
 * rows as they are.  For every param whose bit is set in `bf16_params` (bit
 * i = the i-th sluice_layer_add_param, its rows bf16 values, a multiple of
 * 2048 per row; at most 4 params, the pulled ones excepted) the layer codes
 * each expert's row losslessly into a pinned host store of its own
 * (sluice_codec_encode, on up to 16 host threads): sign and mantissa whole,
 * the exponent as a 4-bit code (its offset in a 14-binade window based per
 * 2048 values; 14 for exponent 0), exponents outside the window in a
 * per-chunk escape list.  A param whose rows code
 * to more than 7/8 of their bytes stays uncoded.  Under a gap server whose
 * gaps are answered before their rows land (sluice_gap_set_pipelined(1)),
 * a miss then copies the coded rows over the link into a ring in HBM that
 * the server owns (at least 128 MiB, and twice the largest coded expert),
 * and a decode kernel, dispatched on an HSA queue of the library's own
 * (sluice_amd/codec_decode.hsaco, beside the library), writes the rows into the
 * slot and marks it ready; staging rows hold coded rows too and are decoded
 * from where they lie.  Slot bytes, maps and products are those of the
 * uncoded store; every other path (inline gaps, classic waves, resync),
 * and a gap server that could not set up its decode resources (no
 * sluice_amd/codec_decode.hsaco beside the library, no HSA queue), copies
 * the rows as they are, from the store given to add_param, which must stay
 * valid.  Call before sluice_layer_set_staging and with no gap
 * server serving the layer; 0 frees the coded stores; a call with the mask
 * already set changes nothing.  SLUICE_E_STATE after staging is set. */
int sluice_layer_set_codec(sluice_layer* layer, uint32_t bf16_params);
/* counters[6]: params coded, bytes of one expert's coded params as rows,
 * bytes of every local expert's coded rows, bytes of the slot fills' row
 * copies over the link (served gaps and classic waves; coded or not),
 * decode jobs launched, and those that decoded a staging row. */
int sluice_layer_codec_counters(const sluice_layer* layer, int64_t* counters);

/* The host store codec by itself.  sluice_codec_encode codes n bf16 values
 * (n a multiple of 2048; rows 2-byte, out 4-byte aligned) into out (cap
 * bytes; NULL to ask) and sets *coded_bytes; sluice_codec_decode decodes
 * `coded_bytes` of a coded row in device memory into n bf16 values at
 * out_dev (both 16-byte aligned) on `stream` and waits for it (it
 * allocates a word of device memory per call). */
int sluice_codec_encode(const void* rows, size_t n, void* out, size_t cap,
                        size_t* coded_bytes);
int sluice_codec_decode(const void* coded_dev, size_t n, size_t coded_bytes,
                        void* out_dev, sluice_stream_t stream);

/* Mark a slot as pre-filled with `local` outside the SLRU segments (full
 * residency pre-fill and static pins, offloader.py:1000-1010, 1046-1083);
 * debits protected_cap by one when `debit_protected` is set (pins). */
int sluice_layer_pin(sluice_layer* layer, int local, int debit_protected,
                     int* slot_out);

/* The gap, split where the host is needed (replaces _router_split_gap,
 * src/sluice/offloader.py:2362-2467, and the ids D2H sync at 2406).
 *
 * Device half, sluice_layer_gap_launch: one workgroup on `stream`, no host
 * call, capturable in a hipGraph.  It builds the step's sorted unique
 * selected ids and the count of owned ids the device map does not hold,
 * posts them to the layer's mailbox (host-mapped pinned memory; the stamp is
 * stored after the record's stores have completed), copies hs_bytes
 * (multiple of 16, 16-byte
 * aligned; 0 = none) from hs_src to hs_dst -- the gap op's fresh copy of
 * hidden_states -- and then waits for the host ONLY if residency must change
 * (a miss, or no standing map yet); it then installs the standing map the
 * host sent.  A step without misses never waits: slots and map stay valid
 * whatever the SLRU bookkeeping does with it.  Device waits are bounded by
 * SLUICE_GAP_TIMEOUT_S (default 20 s) and by the abort flag.
 *
 * Host half, sluice_layer_gap_serve: waits (bounded) for the layer's next
 * record, runs the reference's bookkeeping exactly (fast-hit, hit touches in
 * ascending id order, claimed set, victims), answers the device with the
 * standing slot table and the slots being filled, then streams the misses
 * as SDMA copies through the HSA runtime on two copy lanes (an SDMA engine
 * each; each per-expert param on the lane its layer assigned it, row bytes
 * balanced; the small pulled rows are copied by the gap kernel) and marks
 * each filled slot ready once every copy of its rows completed: the expert
 * product computes resident experts meanwhile and waits per filled slot.  `compute` (may be NULL) is
 * polled for errors while waiting.  SLUICE_E_OVERFLOW when the working set
 * does not fit (rows acquired before it still stream and land before the
 * answer, the map is left as it was, as in the reference).
 *
 * plan (may be NULL): a device buffer of sluice_moe_plan_ints(1, n) ints;
 * the kernel then also builds the expert product's plan of these ids over
 * the map it leaves installed (and its pending slots), for
 * sluice_fused_experts_* to take instead of launching its align kernel.
 *
 * sluice_layer_gap = launch (no copy, no plan) + serve: the reference's
 * eager op. */
int sluice_layer_gap_launch(sluice_layer* layer, const int32_t* topk_ids, int n,
                            const void* hs_src, void* hs_dst, size_t hs_bytes,
                            int32_t* plan, sluice_stream_t stream);
int sluice_layer_gap_serve(sluice_layer* layer, int fast_hit,
                           sluice_stream_t compute);
int sluice_layer_gap(sluice_layer* layer, const int32_t* topk_ids, int n,
                     int fast_hit, sluice_stream_t compute);

/* Gap server: a native thread that serves every listed layer's records as
 * the device posts them, so the gap op needs no host code on the stream and
 * a whole decode step (gaps included) can replay as one hipGraph.  While a
 * layer is served, sluice_layer_gap/_serve/_gap_host on it return
 * SLUICE_E_STATE.  On the first error the server raises the abort flag
 * (waiting gap kernels exit, maps unchanged) and keeps it as its sticky
 * error.  drain: after the caller has synchronised the streams that launched
 * gaps, waits until every posted record is served; returns the sticky error.
 * No counterpart in the reference (its gap is always eager). */
typedef struct sluice_gap_server sluice_gap_server;
int sluice_gap_server_create(sluice_layer* const* layers, int n_layers,
                             int fast_hit, sluice_gap_server** out);
int sluice_gap_server_drain(sluice_gap_server* server, double timeout_s);
int sluice_gap_server_error(const sluice_gap_server* server);
int sluice_gap_server_destroy(sluice_gap_server* server);

/* Raise (set=1) or clear (set=0) the process-wide abort flag; after an abort
 * and a stream synchronisation, sluice_layer_gap_resync lines a layer's host
 * stamps up with the device's. */
int sluice_gap_abort(int set);

/* The bound of the gap's waits (device and host), in seconds; 0 restores
 * SLUICE_GAP_TIMEOUT_S (default 20).  The device waits read the bound from
 * a per-device word when they begin, so it applies to every wait that
 * begins after the call, in direct launches and in graphs captured before
 * it alike.  No counterpart in the reference (its gap waits are host syncs
 * without a bound); it lets callers, and tests, shorten a wait that must
 * end. */
int sluice_gap_set_timeout(double seconds);

/* on=1 (default): a gap that streams misses is answered before the rows
 * land and the expert product waits per filled slot.  on=0: the answer
 * waits until every row landed, the order of the reference's gap, whose
 * compute stream waits for the copy event before the expert product
 * (src/sluice/offloader.py:2464, 1986-1991); slot assignment, maps and
 * outputs are the same either way.  Applies to records served after the
 * call. */
int sluice_gap_set_pipelined(int on);

/* After an abort or a failed gap, once every stream that ran the layer's
 * gap kernels is synchronised: drains the copy lanes, lines the host's
 * stamps up with the device's, clears the pending-slot marks and writes the
 * host's standing map into the device map (which may lag the slot cache:
 * a device wait that ended after the host served its record, or fills
 * dropped after a failed copy).  It also copies again the rows the gap
 * kernel copies itself (sluice_layer_pulled_params) into every slot the
 * cache holds: a gap the host answered but the device never installed left
 * them out.  No counterpart in the reference, whose gap errors end the
 * engine. */
int sluice_layer_gap_resync(sluice_layer* layer);

/* Recovery from a fill whose rows did not land: the expert in `slot` leaves
 * the slot cache (its segment, slot_of, expert_in_slot), the slot goes back
 * on the free list (taken next) and the map stops being the standing map,
 * so the next gap selecting the expert misses and streams it again.  The
 * served gap does this itself for every fill of a failed stream-in that was
 * not seen to land.  SLUICE_E_STATE for an empty or pinned slot.  No
 * counterpart in the reference (its copy errors end the engine). */
int sluice_layer_unfill(sluice_layer* layer, int slot);

/* Failure injection for tests of the recovery path, forced from the host:
 * the (after+1)-th row copy a served gap issues from now on is not issued
 * and reports hipErrorInvalidValue, once; after < 0 disarms.  Every kernel
 * still exits normally (the failed gap's slots are marked ready, the
 * failure is reported).  No counterpart in the reference. */
int sluice_gap_inject_copy_failure(int after);

/* Gap timeline tracing, for the -DSLUICE_TRACE build only (every call
 * returns SLUICE_E_STATE in the default build).  The gap kernel, the expert
 * product's split launch and the combine stamp events with the device wall
 * clock; the host gap service stamps its steps with CLOCK_MONOTONIC.
 * sluice_trace_read: which 0 = gap kernel ring, 1 = expert product ring
 * (both 2^20 records of {tag << 56 | value, wall clock}, 16 bytes), 2 = host
 * ring (2^18 records {uint32 tag, uint32 layer, int32 stamp, int32 value,
 * double seconds}); *n = records written since the last reset (a ring keeps
 * its last 2^20 or 2^18); out may be NULL.  sluice_trace_calibrate: n pairs of
 * (host seconds, device wall-clock ticks mod 2^48) of the same instants up to
 * the bus latency; returns the pairs taken.  No counterpart in the
 * reference; diagnostics only. */
int sluice_trace_calibrate(int n, double* host_s, unsigned long long* dev_ticks);
int sluice_trace_read(int which, void* out, unsigned* n);
int sluice_trace_reset(void);

/* The gap, host path (no HIP calls): ids is a host array.  Runs the same
 * bookkeeping and reports the (local, slot) stream-ins in order in
 * streams[2*i], streams[2*i+1] (capacity 2*max_streams ints) and whether
 * the standing map would be rewritten (*map_written). */
int sluice_layer_gap_host(sluice_layer* layer, const int32_t* ids, int n,
                          int fast_hit, int32_t* streams, int max_streams,
                          int* n_streams, int* map_written);

/* Classic (wave) step: replaces run_moe (src/sluice/offloader.py:1452-1765)
 * and _run_waves (1846-1933), the path of steps the gap does not take (more
 * tokens than the router-split envelope, prefill chunks).
 *
 * sluice_layer_classic_plan: copies topk_ids [n] (int32, device, row-major
 * [T, n/T]) to the host on `stream` and synchronises it (the reference's one
 * host sync per layer, 1540); with a gap server attached, waits until the
 * layer's posted gap records are served; then runs the reference's
 * bookkeeping exactly: decode classification from nd / ndec (< 0 = not
 * published) / real_step / spec_tokens, class-aware touches and fills,
 * decode-class misses first, leftover misses rotated through the probation
 * slots in two ping-pong groups.  *n_waves >= 1.  Refuses a capturing
 * stream (SLUICE_E_STATE).  The map stops being the standing map; the
 * layer's next gap reinstalls it.
 *
 * Then, for w = 0 .. n_waves-1, the caller enqueues the expert product on
 * `stream` between sluice_layer_classic_wave(w) -- writes wave w's map
 * (its (global, slot) pairs, -1 elsewhere), and makes `stream` wait for the
 * wave's row copies, which run on the library's copy lanes (wave 0's after
 * the work already on `stream`) -- and sluice_layer_classic_wave_done(w),
 * which records the wave's end and issues wave w+1's copies behind the
 * kernel that last read those slots.  The caller sums the wave outputs.
 * Waves must run in order; a plan left unfinished has its remaining copies
 * issued by the next plan. */
int sluice_layer_classic_plan(sluice_layer* layer, const int32_t* topk_ids,
                              int n, int T, int nd, int ndec, int real_step,
                              int spec_tokens, sluice_stream_t stream,
                              int* n_waves);
int sluice_layer_classic_wave(sluice_layer* layer, int wave,
                              sluice_stream_t stream);
int sluice_layer_classic_wave_done(sluice_layer* layer, int wave,
                                   sluice_stream_t stream);

/* The classic step's bookkeeping on host ids (no HIP calls). */
int sluice_layer_classic_host(sluice_layer* layer, const int32_t* ids, int n,
                              int T, int nd, int ndec, int real_step,
                              int spec_tokens, int* n_waves);

/* The last classic plan: out = [n_waves, pipelined, then per wave: n_pairs,
 * n_pairs x (global, slot), n_streams, n_streams x (local, slot)]; *len is
 * its length (out may be NULL to size it).  counters[2] (may be NULL) =
 * {classic steps, classic waves}. */
int sluice_layer_classic_plan_read(const sluice_layer* layer, int32_t* out,
                                   int cap, int* len, int64_t* counters);

/* Opt-in policies of the slot cache, both off by default.
 *   lfu (SLUICE_LFU, src/sluice/offloader.py:1993-2007, 2023-2034,
 *     2057-2068): real classic steps count each selected local expert; the
 *     counts are halved every 256 such steps; while any count is nonzero the
 *     protected segment demotes, and gives up victims, least frequent first
 *     (LRU among equals).
 *   count_experts (SLUICE_EXPERT_COUNTS, 1026-1034, 1664-1671): real classic
 *     steps count each selected global expert as decode-class or scan-class.
 * sluice_layer_policy_state: freq [local_n], counts_decode / counts_scan [E]
 * (each may be NULL); stats[3] = {pure-decode ("small") classic steps, scan
 * classic steps, steps since the last LFU halving}. */
int sluice_layer_set_policy(sluice_layer* layer, int lfu, int count_experts);
int sluice_layer_policy_state(const sluice_layer* layer, int64_t* freq,
                              int64_t* counts_decode, int64_t* counts_scan,
                              int64_t* stats);

/* Classic-step stats by class, as the reference's get_stats() buckets them
 * (src/sluice/offloader.py:172-183, 1656-1684, 1711-1713, 1887, 2804-2814):
 * out[8] = {small: steps, hits, misses, waves, scan: steps, hits, misses,
 * waves}, real steps only ("small" = pure decode).  Bytes streamed are
 * misses x bytes per expert. */
int sluice_layer_step_stats(const sluice_layer* layer, int64_t* out);

/* State snapshot.  Arrays may be NULL.  slot_of [local_n] (-1 = absent),
 * expert_in_slot [S] (-1 = empty), probation/protected in recency order
 * (LRU first), free_slots in list order (the last is popped next).
 * counters[8] = {gaps, misses, fast_hits, map_writes, bytes_lo, bytes_hi,
 *                map_is_standing, protected_cap}. */
int sluice_layer_state(const sluice_layer* layer, int32_t* slot_of,
                       int32_t* expert_in_slot, int32_t* probation,
                       int* n_probation, int32_t* protected_, int* n_protected,
                       int32_t* free_slots, int* n_free, int64_t* counters);

/* The standing map the layer would publish (host [E] int32). */
int sluice_layer_standing_map(const sluice_layer* layer, int32_t* map_out);

#ifdef __cplusplus
}
#endif

#endif /* SLUICE_H_ */
