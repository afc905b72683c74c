/* cfhip.h -- C ABI of the MI355X (gfx950) chain-flow drafting hot path (libcfhip.so).
 *
 * Every entry point takes plain device pointers and sizes, an explicit HIP stream (hipStream_t
 * passed as void*; NULL = the null stream) and returns 0 (CFH_OK) or an error code
 * (cfh_error_string() names it).  Nothing here allocates device memory: callers own the weights,
 * the workspace and the outputs.  All launches are asynchronous on the given stream and may be
 * recorded into a HIP graph (no memset nodes).  One exception to "no host synchronisation": the
 * first eager cfh_flow_integrate on a caller stream (for flows whose chunk experts run
 * concurrently) creates that stream's companion streams and events and checks once, with a
 * synchronisation of the caller's stream, that they run alongside it; cfh_flow_prepare_streams
 * does that at set-up time instead, and nothing under stream capture ever does it.
 *
 * The reference (Cosmos-YTU/chain-flow, `cf/` = src/chain_flow/) binds its hot path through a
 * pybind torch extension (cf/csrc/fused_block.cu:793-862) plus plain torch ops; each entry point
 * below says which reference interface it replaces.
 *
 * fp16 = IEEE half, bf16 = bfloat16; "packed" = the MFMA tile order produced by cfh_pack_linear.
 */
#ifndef CFHIP_H
#define CFHIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CFH_OK 0
#define CFH_E_INVALID 1          /* bad argument (null pointer, size out of range)        */
#define CFH_E_UNSUPPORTED 2      /* shape this build does not support                     */
#define CFH_E_HIP 3              /* a HIP runtime call failed (cfh_last_hip_error)        */
#define CFH_E_SCRATCH 4          /* the no-allocation entry point's workspace is too small */

/* Size of the library's per-device scratch array behind cfh_flow_integrate_noalloc (64 MiB: the
 * flow workspace of one request at d <= 5120 and 8 layers needs 35.9 MiB; a batch packs two
 * requests per group where the shape allows, which can need more -- cfh_caps tells). */
#define CFH_NOALLOC_SCRATCH_BYTES (64ll << 20)

/* Library version (major*10000 + minor*100 + patch). */
int cfh_version(void);
/* Human-readable text for a status code. */
const char* cfh_error_string(int status);
/* The hipError_t of the last failing HIP call made by this library on this thread. */
int cfh_last_hip_error(void);

/* ---------------------------------------------------------------- weight packing
 * Pack a row-major linear weight W[n][k] (nn.Linear layout, fp16 or bf16 -- the packing is
 * dtype-agnostic 2-byte data) into MFMA tile order: out holds n*k halves.  n % 16 == 0,
 * k % 32 == 0.  Replaces the reference's host-side weight packing
 * (cf/cuda_block.py:269-318, layout cf/csrc/fused_block.cu:47-79). */
int cfh_pack_linear(const void* w, int n, int k, void* out, void* stream);

/* ---------------------------------------------------------------- flow (velocity net + Euler)
 * Shape of one TreeFlowDrafter flow: HiddenKVFlowExpert chunk experts
 * (cf/drafters/tree_flow.py:40-77, cf/drafters/chunked_flow.py:205-414). */
typedef struct cfh_flow_dims {
  int d;             /* expert_dim: the target hidden size, or the VAE latent size (640 /  */
                     /* 1024) in the latent drafters; d % 64 == 0, d <= 16384             */
  int ffn_mult;      /* ffn multiplier (6)                                                 */
  int heads;         /* attention heads (8); head width d / heads a multiple of 8 (80 at  */
                     /* d = 640: two heads share an MFMA k-chunk)                          */
  int layers;        /* HiddenKVFlowBlocks per expert (num_drafter_layers)                 */
  int ctx_rows;      /* context_size (8); 2 <= ctx_rows <= 16                              */
  int draft_length;  /* draft_length (8); <= 16                                            */
  int chunk_size;    /* chunk_size (4); draft_length % chunk_size == 0                     */
  int flow_steps;    /* num_flow_steps E (Euler steps); 1 <= E <= 16                       */
  int numerics;      /* CFH_FLOW_FUSED or CFH_FLOW_MODULES: the rounding points to follow      */
  int init_mode;     /* CFH_INIT_DELTA, CFH_INIT_REPEAT_LAST or CFH_INIT_GIVEN (init_latents) */
} cfh_flow_dims;

/* The initial latents z0 of the Euler integration, per request (init_latents,
 * cf/drafters/tree_flow.py:150-161), from the fp16 context rows c[0..C-1]:
 *   CFH_INIT_DELTA        z0[k] = fp16(c[C-1] + fp16((k+1) * fp16(c[C-1] - c[C-2])))  ("delta")
 *   CFH_INIT_REPEAT_LAST  z0[k] = c[C-1]                                              ("repeat_last")
 *   CFH_INIT_GIVEN        z0 is read from z_out on entry ([batch][draft_length][d] fp16): for the
 *                         reference's "noise" mode the caller draws randn(...) * noise_scale with
 *                         its own generator, as the reference does. */
#define CFH_INIT_DELTA 0
#define CFH_INIT_REPEAT_LAST 1
#define CFH_INIT_GIVEN 2

/* The two fp16 numerics the reference runs its flow blocks in (both with fp32 accumulation, fp16
 * q/k/v, attention and LayerNorm outputs):
 *   CFH_FLOW_FUSED   its fused block kernel (cf/csrc/fused_block.cu:280-325, 452-668), engaged
 *                    for D in {640, 1024}, ffn x6, 8 heads, chunk rows in {4, 8}, <= 16 context
 *                    rows, batch 1 (cf/cuda_block.py:95-102, cf/drafters/chunked_flow.py:
 *                    295-331): fp32 residual stream, GELU of the fp32 pre-activation;
 *   CFH_FLOW_MODULES torch's fp16 modules, every other shape (cf/drafters/chunked_flow.py:185-202):
 *                    fp16 residual stream x = fp16(x + fp16(sublayer)), GELU of the
 *                    fp16-rounded up-projection. */
#define CFH_FLOW_FUSED 0
#define CFH_FLOW_MODULES 1

/* Capability/shape gate: 0 (CFH_OK) if this build runs `dims` at `batch`, with the workspace
 * size in *ws_bytes; CFH_E_UNSUPPORTED otherwise.  Replaces cuda_block.supported()/max_grid()
 * (cf/cuda_block.py:95-163, cf/csrc/fused_block.cu:836-856). */
int cfh_caps(const cfh_flow_dims* dims, int batch, int64_t* ws_bytes);

/* Bytes of one expert's packed weight image. */
int64_t cfh_flow_expert_bytes(const cfh_flow_dims* dims);

/* Pack one chunk expert.  raw[] = device pointers to the expert's fp16 parameters in
 * state_dict order (n_raw = 9 + 20*layers):
 *   position_embedding.weight, time_mlp.0.weight, time_mlp.0.bias, time_mlp.2.weight,
 *   time_mlp.2.bias, then per block l: self_norm.{weight,bias}, self_attn.in_proj_{weight,bias},
 *   self_attn.out_proj.{weight,bias}, cross_norm.{weight,bias}, context_norm.{weight,bias},
 *   cross_attn.in_proj_{weight,bias}, cross_attn.out_proj.{weight,bias}, ffn.0.{weight,bias},
 *   ffn.1.{weight,bias}, ffn.4.{weight,bias}, then out_norm.{weight,bias}, out_proj.{weight,bias}.
 * The image also holds the time embeddings of every Euler step (time_mlp(s / flow_steps), a function
 * of the weights alone), which packing computes on `stream`.
 * Replaces FusedExpertBlocks.__init__ packing (cf/cuda_block.py:269-318). */
int cfh_flow_pack_expert(const cfh_flow_dims* dims, const void* const* raw, int n_raw, void* packed,
                         void* stream);

/* TreeFlowDrafter.predict_hidden (cf/drafters/tree_flow.py:229-244): init_latents(ctx) then all
 * E Euler steps of both chunk experts (every block of every expert, cross-K/V hoisted once).
 *   experts : n_chunks = draft_length/chunk_size packed expert images (chunk order)
 *   ctx     : [batch][ctx_rows][d] fp16 context hidden states (already front-padded)
 *   z_out   : [batch][draft_length][d] fp16 predicted hiddens
 *   ws      : workspace of cfh_caps(dims, batch) bytes
 * A batch runs in groups of requests whose rows share every weight stream: up to sixteen (wide
 * groups, rows staged in K chunks; head width a multiple of 128 and the folded cross attention),
 * else up to two (both drafts in one 16-row MFMA tile); cfh_flow_group_size tells.
 * Chunk experts (d >= 1024, two or more chunks) run their Euler steps on companion streams of the
 * caller's stream, forked after the per-draft launches and joined before return.  The first eager
 * call on a caller stream without companions creates them (streams, events: kept until
 * cfh_flow_release_streams) and runs the overlap check of cfh_flow_prepare_streams, which
 * synchronises the caller's stream once; under stream capture every expert stays on the caller's
 * stream and nothing is created.  Same results on one stream or several, bit for bit.
 * Replaces the per-Euler-step torch loop plus the fused kernel launch
 * (cf/cuda_block.py:407-431 / pybind `expert`, `cross_kv`, cf/csrc/fused_block.cu:793-862) and the
 * reference's two-stream chunk pair (cf/cuda_block.py:452-466). */
int cfh_flow_integrate(const cfh_flow_dims* dims, const void* const* experts, const void* ctx,
                       void* z_out, void* ws, int batch, void* stream);

/* The anchored latent drafter (TreeVAEFlowConfig.anchor_token): the embedding of each request's
 * committed token, through the drafter's anchor_in and each chunk expert's anchor_mlp, conditions
 * every row of every block (cf/drafters/tree_flow.py:237-241, cf/drafters/chunked_flow.py:256-262,
 * 376: x = fp16(x + anchor_mlp(anchor)) after the position and time embeddings):
 *   cfh_flow_anchor: anchor[c][b] = fp16(W2_c fp16(silu(fp16(W1_c t_b + b1_c))) + b2_c) with
 *     t_b = fp16(W_in embed_w[max(tokens[b], 0)] + b_in); aw = 2 + 4 n_chunks device pointers:
 *     anchor_in.weight (PACKED, [d][hidden]), anchor_in.bias, then per chunk expert
 *     anchor_mlp.0.weight (PACKED [d][d]), anchor_mlp.0.bias, anchor_mlp.2.weight (PACKED), anchor_mlp.2.bias;
 *     embed_w [V][hidden] fp16, tokens [batch] int32, anchor [n_chunks][batch][d] fp16 out,
 *     ws of cfh_flow_anchor_ws_bytes bytes.
 *   cfh_flow_integrate_anchored: cfh_flow_integrate with those rows added (the reference's
 *     predict_hidden(ctx, anchor_embed(known0)), flow_proposer.py:1203, 1285). */
int64_t cfh_flow_anchor_ws_bytes(const cfh_flow_dims* dims, int hidden);
int cfh_flow_anchor(const cfh_flow_dims* dims, int hidden, const void* const* aw, const void* embed_w,
                    const int32_t* tokens, int batch, void* anchor, void* ws, void* stream);
int cfh_flow_integrate_anchored(const cfh_flow_dims* dims, const void* const* experts, const void* ctx,
                                const void* anchor, void* z_out, void* ws, int batch, void* stream);

/* Requests per group (*requests) that cfh_flow_integrate drafts together for a batch of `batch`:
 * every weight byte streams once per group.  No counterpart in the reference, whose batched flow
 * runs torch modules over the whole batch (cf/drafters/chunked_flow.py:295-331). */
int cfh_flow_group_size(const cfh_flow_dims* dims, int batch, int* requests);

/* The launch forms cfh_flow_integrate uses for `batch` requests of this shape (*flags, bits below):
 * a diagnostic with no counterpart in the reference, for callers and tests that need to know which
 * kernels a shape runs.  Host only: touches no device. */
#define CFH_PLAN_FOLD 1      /* cross attention folded into per-draft factors (k_xattn)                 */
#define CFH_PLAN_FOLD2 2     /* ... with two heads a k-chunk (head widths such as 80)                   */
#define CFH_PLAN_XBLK 4      /* residual rows and folded cross attention in one launch a block pass     */
#define CFH_PLAN_WIDE 8      /* wide request groups (more than two requests share each weight stream)   */
#define CFH_PLAN_CONC 16     /* chunk experts on companion streams (when the overlap check passes)      */
int cfh_flow_plan(const cfh_flow_dims* dims, int batch, int* flags);

/* Set-up of the companion streams of a caller stream, so that no later cfh_flow_integrate on it
 * synchronises: creates the companions `dims`'s chunk experts need (none for flows that stay on one
 * stream) and checks once that work on them overlaps work on the caller's stream (two 200 us wait
 * kernels, then a synchronisation of the caller's stream).  HIP maps a process's streams onto a
 * few hardware queues, and streams that share one run in submission order: then the flow keeps
 * every expert on the caller's stream.  *concurrent = 1 when the experts will run concurrently.
 * CFH_E_INVALID under stream capture.  Mirrors the reference's side-stream set-up for its chunk
 * pair (cf/cuda_block.py:452-466). */
int cfh_flow_prepare_streams(const cfh_flow_dims* dims, void* stream, int* concurrent);
/* The companions of a caller stream on the current device: how many exist, and whether the flow
 * runs its chunk experts on them (the overlap check passed).  Creates nothing. */
int cfh_flow_query_streams(void* stream, int* companions, int* concurrent);
/* Destroys the companions of a caller stream (their queued work completes first).  Call it before
 * destroying the caller's stream: the companions are keyed by the stream handle, and a later
 * stream that reuses the handle would inherit their overlap verdict.  Not concurrently with a
 * flow call on that stream. */
int cfh_flow_release_streams(void* stream);

/* cfh_flow_integrate without a caller workspace, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  It has no
 * counterpart in the reference.  The workspace is the library's file-scope device array of
 * CFH_NOALLOC_SCRATCH_BYTES, one per device, resolved on the first call on each device; nothing
 * is allocated or freed.  Shapes whose workspace (cfh_caps) exceeds it return CFH_E_SCRATCH.
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU (two streams, two
 * host threads) race and must be serialised by the caller.  It creates no stream or event either:
 * the chunk experts run on companion streams only if an earlier cfh_flow_integrate call on the
 * same caller stream created them, else all on the caller's stream.  Same results as
 * cfh_flow_integrate. */
int cfh_flow_integrate_noalloc(const cfh_flow_dims* dims, const void* const* experts, const void* ctx,
                               void* z_out, int batch, void* stream);

/* ---------------------------------------------------------------- hidden-state VAE
 * TransformerHiddenVAE (cf/vae/transformer_hidden.py:9-79; config cf/vae/base.py:9-17): the frozen
 * VAE the latent drafters run the flow inside (cf/drafters/tree_vae_flow.py:163-175).  Each half is
 * input Linear + position embedding, `layers` pre-LN nn.TransformerEncoderLayers (bidirectional
 * self-attention, GELU FFN of 4*inter, LayerNorm eps 1e-5), a final LayerNorm and an output
 * Linear, in fp16 with the rounding points of torch's fp16 modules (fp16 residual stream). */
typedef struct cfh_vae_dims {
  int hidden;        /* target hidden size (encoder input, decoder output); % 64 == 0     */
  int latent;        /* latent_size (640 / 1024); % 64 == 0                               */
  int inter;         /* intermediate_size (1920): transformer width; % 64 == 0            */
  int layers;        /* num_layers of each half (2)                                       */
  int heads;         /* num_heads (8); 1 when inter % num_heads != 0, as the module does  */
  int max_rows;      /* max_sequence_length (16): rows of the position tables             */
} cfh_vae_dims;

/* Bytes of the packed VAE image (-1 if `dims` is unsupported). */
int64_t cfh_vae_bytes(const cfh_vae_dims* dims);

/* Pack the VAE.  raw[] = device pointers to its fp16 parameters in state_dict order, logvar
 * omitted (n_raw = 14 + 24*layers):
 *   encoder_in.{weight,bias}, encoder_pos.weight, per encoder layer l:
 *   encoder.layers.l.self_attn.in_proj_{weight,bias}, .self_attn.out_proj.{weight,bias},
 *   .linear1.{weight,bias}, .linear2.{weight,bias}, .norm1.{weight,bias}, .norm2.{weight,bias},
 *   then encoder_norm.{weight,bias}, mu.{weight,bias}, decoder_in.{weight,bias},
 *   decoder_pos.weight, the decoder layers in the same order, decoder_norm.{weight,bias},
 *   decoder_out.{weight,bias}.
 * Replaces _load_frozen_vae's module build (cf/drafters/tree_vae_flow.py:50-87). */
int cfh_vae_pack(const cfh_vae_dims* dims, const void* const* raw, int n_raw, void* packed, void* stream);

/* 0 if this build runs `dims` on sequences of `rows` rows (rows <= 16 and <= max_rows), with the
 * workspace size in *ws_bytes (enough for any batch: a batch of sequences runs in groups of up to
 * 128 / rows sequences stacked, one launch sequence a group); CFH_E_UNSUPPORTED otherwise. */
int cfh_vae_caps(const cfh_vae_dims* dims, int rows, int64_t* ws_bytes);

/* encode_sequence(hidden).mu (cf/vae/transformer_hidden.py:52-59): hidden [batch][rows][hidden]
 * fp16 -> mu [batch][rows][latent] fp16.  Replaces TreeVAEFlowDrafter._encode (tree_vae_flow.py:
 * 163-165). */
int cfh_vae_encode(const cfh_vae_dims* dims, const void* packed, const void* hidden, void* mu, int batch,
                   int rows, void* ws, void* stream);

/* decode_sequence(z) (cf/vae/transformer_hidden.py:61-68): z [batch][rows][latent] fp16 ->
 * out [batch][rows][hidden] fp16.  Replaces TreeVAEFlowDrafter._decode (tree_vae_flow.py:167-169). */
int cfh_vae_decode(const cfh_vae_dims* dims, const void* packed, const void* z, void* out, int batch,
                   int rows, void* ws, void* stream);

/* ---------------------------------------------------------------- context ring
 * FlowDrafterProposer._ring_write + _ring_gather (cf/vllm_plugin/flow_proposer.py:916-961) as one
 * launch, one workgroup per request.  ring [R][C+1][H] (2-byte elements; row C is the reference's
 * trash row, unused), rpos / nval [R] int32 = next write position / valid rows per slot.
 * For request b (slot rows[b]): rows j < min(cnt[b], Kmax) of sh [T][H] (same element type as the
 * ring) at starts[b] + j -- or, with a tree's accepted path [R][path_ld], at starts[b] + 0 and
 * starts[b] + 1 + path[slot][j-1] -- are appended unless wmask[b] == 0 (wmask NULL = all 1);
 * rpos/nval advance; then, if ctx [B][C][H] is set, the slot's window is read back oldest first,
 * front-padded by repeating the oldest row (TreeFlowDrafter._context, tree_flow.py:143-148).
 * cnt NULL = gather only.  H % 8 == 0. */
int cfh_ring_step(void* ring, int32_t* rpos, int32_t* nval, int C, int H, const void* sh, int T,
                  const int32_t* rows, const int32_t* starts, const int32_t* cnt, const int32_t* wmask,
                  const int32_t* path, int path_ld, int Kmax, int B, void* ctx, void* stream);

/* ---------------------------------------------------------------- shortlisted lm_head
 * logits[m][j] = fp16( fp16(h[m] . W[row_j]) + fp16(A[m] . W2[row_j]) ),  row_j = sl ? sl[j] : j
 *   h [M][d] fp16 (M <= 8, d % 256 == 0); W [V][d] fp16: the target's full lm_head, its shortlist
 *   rows read in place through the int32 shortlist sl [n] (no gathered copy of lm_w[sl]);
 *   markov bias (a, W2 NULL = none): A[m] = a[a_ids[m * a_ids_stride]] when a_ids is set (a = the
 *   w1 table [V][r]) else a[m] ([M][r] fp16); W2 [V][r] fp16, r % 256 == 0.  logits [M][n] fp16.
 * Replaces FlowDrafterProposer._head + _bias (cf/vllm_plugin/flow_proposer.py:1021-1025, 739-740). */
int cfh_head_logits(const void* h, int M, int d, const void* W, const int32_t* sl, int n,
                    const void* a, const int32_t* a_ids, int a_ids_stride, int r, const void* W2,
                    void* logits, void* stream);

/* Per-row log-softmax top-k of fp16 logits [M][n]: vals[m][i] = logit - logsumexp (fp32),
 * ids[m][i] = column, descending, ties to the lower column; lse[m] (may be NULL).  k <= 16.
 * Replaces torch.log_softmax(logits.float()).topk(k) (cf/vllm_plugin/flow_proposer.py:1249-1250). */
int cfh_row_topk(const void* logits, int M, int n, int k, float* vals, int32_t* ids, float* lse,
                 void* stream);

/* Bytes of the candidate workspace `ws` that cfh_head_topk / cfh_head_gemm_topk need for M rows,
 * n shortlist columns and top-k (-1 if out of range). */
int64_t cfh_head_ws_bytes(int M, int n, int k);

/* cfh_head_logits with the log-softmax top-k fused into the head: every workgroup reduces its
 * column block to per-row (max, sum-exp) and a local top-k in `ws`, a merge kernel combines them.
 * `logits` [M][n] fp16 is an optional output (NULL: the logits never reach memory).
 * Same results as cfh_head_logits followed by cfh_row_topk. */
int cfh_head_topk(const void* h, int M, int d, const void* W, const int32_t* sl, int n,
                  const void* a, const int32_t* a_ids, int a_ids_stride, int r, const void* W2, int k,
                  void* logits, float* vals, int32_t* ids, float* lse, void* ws, void* stream);

/* Bytes of the packed shortlist head image for n shortlist columns, dimension d and markov rank r
 * (0: no markov table); -1 if out of range. */
int64_t cfh_head_packed_bytes(int n, int d, int r);

/* Gathers the shortlisted rows W[sl[j]] (and W2[sl[j]] when r > 0) into one image in the MFMA
 * fragment order, once per shortlist: the layout-for-bandwidth form of the in-place row gather of
 * cfh_head_topk (cf/vllm_plugin/flow_proposer.py:1021-1025 reads lm_head[shortlist] per call).
 * packed: cfh_head_packed_bytes(n, d, r) bytes.  sl NULL = rows 0..n-1. */
int cfh_head_pack(const void* W, const void* W2, const int32_t* sl, int n, int d, int r, void* packed,
                  void* stream);

/* cfh_head_topk over a cfh_head_pack image (no sl, W, W2: the image holds them).  Same results. */
int cfh_head_topk_packed(const void* h, int M, int d, const void* packed, int n, const void* a,
                         const int32_t* a_ids, int a_ids_stride, int r, int k, void* logits, float* vals,
                         int32_t* ids, float* lse, void* ws, void* stream);

/* Pass A of the two-pass candidate head (FlowDrafterProposer._candidates, flow_proposer.py:
 * 1142-1165): for each of B requests owning n consecutive rows of fp16 logits [B*n][ld] (over Vs
 * shortlist columns) with their log-sum-exp lse [B*n], value[j] = max_d (logits[d][j] - lse[d]);
 * the M columns of largest value (ties to the lower column), ascending, into cand_local [B][M] and,
 * mapped through the shortlist sl (NULL = identity), cand_global [B][M] (may be NULL).  n = 1
 * selects per row (the per-depth sets).  ws: cfh_cand_ws_bytes(B, Vs) bytes, 16-byte aligned
 * (CFH_E_INVALID otherwise).  Vs <= 262,144 (CFH_E_UNSUPPORTED above). */
int64_t cfh_cand_ws_bytes(int B, int Vs);
int cfh_cand_topm(const void* logits, long long ld, const float* lse, int B, int n, int Vs, int M, const int32_t* sl,
                  int32_t* cand_local, int32_t* cand_global, void* ws, void* stream);

/* Batched (M up to 256) bf16 skinny-GEMM head with per-row log-softmax top-k: the two-pass
 * candidate head's pass A (cf/vllm_plugin/flow_proposer.py:1142-1165) as one MFMA kernel plus the
 * candidate merge.  logits[m][j] = bf16(x[m] . W[row_j]), row_j = sl ? sl[j] : j.
 *   x [M][d] bf16 (d % 128 == 0), W [V][d] bf16 read in place through sl,
 *   logits [M][n] bf16 optional output (NULL: not written), vals/ids [M][k], lse [M] (may be NULL),
 *   ws of cfh_head_ws_bytes(M, n, k) bytes.  k <= 16. */
int cfh_head_gemm_topk(const void* x, int M, int d, const void* W, const int32_t* sl, int n, int k,
                       void* logits, float* vals, int32_t* ids, float* lse, void* ws, void* stream);

/* cfh_head_gemm_topk over a cfh_head_pack image of W (r = 0; the image holds the shortlist rows,
 * d % 256 == 0): every weight load is a contiguous MFMA fragment.  Same results. */
int cfh_head_gemm_topk_packed(const void* x, int M, int d, const void* packed, int n, int k, void* logits,
                              float* vals, int32_t* ids, float* lse, void* ws, void* stream);

/* cfh_head_topk for G requests at once, each with its own rows and its own shortlist: request g
 * scores its M rows h + g M d (M <= 8) against the n rows sl + g sl_stride (global ids into W and
 * W2, read in place), with the markov rows a_ids + g M a_ids_stride (or A rows a + g M r); the
 * per-row top-k over those n columns goes to rows g M .. g M + M - 1 of vals/ids/lse (ids are
 * positions in that request's list).  ws: cfh_head_ws_bytes(G M, n, k) bytes.  The two-pass head's
 * pass B for a batch (_gather_cand + _rescore, cf/vllm_plugin/flow_proposer.py:1167-1184, a bmm
 * over per-request candidate rows) in one launch. */
int cfh_head_topk_grouped(const void* h, int G, int M, int d, const void* W, const int32_t* sl, long long sl_stride,
                          int n, const void* a, const int32_t* a_ids, int a_ids_stride, int r, const void* W2, int k,
                          float* vals, int32_t* ids, float* lse, void* ws, void* stream);

/* The drafter's fp16 form of the batched head, over a cfh_head_pack image (d % 256 == 0; an image
 * packed with markov rows works too: its lm_head rows come first, and its markov w2 rows start at
 * byte ((n + 15) / 16) * 16 * d * 2 as an r-column image of their own):
 *   logits[m][j] = fp16( fp16(x[m] . W[row_j]) + bias[m][j] )   (bias [M][n] fp16, or NULL: no add)
 * x [M][d] fp16, M <= 256.  k >= 1: the per-row log-softmax top-k into vals/ids/lse (ws of
 * cfh_head_ws_bytes(M, n, k)), logits [M][n] fp16 optional; k = 0: the logits alone (required).
 * With bias = the k = 0 logits of the markov rows against A[m] = w1[prev[m]], the logits are the GEMV
 * head's fp16(fp16(h.W) + fp16(A.W2)).  Replaces the proposer's batched `_head` + `_bias` and
 * log_softmax / topk over B*n rows (cf/vllm_plugin/flow_proposer.py:1021-1025, 1142-1165). */
int cfh_head_gemm16_topk(const void* x, int M, int d, const void* packed, int n, const void* bias, int k,
                         void* logits, float* vals, int32_t* ids, float* lse, void* ws, void* stream);

/* ---------------------------------------------------------------- draft search
 * Path-conditioned residual of the PathHead, fused form (cf/vllm_plugin/fused.py:25-37;
 * un-fused twin cf/drafters/tree_flow.py:434-450):
 *   hsum[m] = fp16( pred_m + MLP(LN( fp16(sum_{j<nlive} mask_j fp16(W_j emb(lastp[m][j]) + b_j)) )) )
 * with emb = embed_w rows [V][d] of the global ids in lastp [M][order] (int32, -1 = no ancestor,
 * mask_j = lastp[m][j] >= 0), nlive = live offsets at this depth (_nlive, :1030-1037).
 * ph = path head fp16 parameters (2*order + 6 device pointers), matrices PACKED (cfh_pack_linear):
 *   offset_proj.{0..order-1}.weight [d][d], offset_proj.{0..order-1}.bias [d], norm.weight,
 *   norm.bias, mlp.0.weight [f*d][d], mlp.0.bias [f*d], mlp.3.weight [d][f*d], mlp.3.bias [d].
 * pred_m fp16 = the marginal hidden of this depth for row m's request: pred + (m / rows_per_pred) *
 * pred_ld (rows_per_pred = 0: every row uses pred[0..d)), so B requests' beams go in one call.
 * Any M >= 1: rows are processed 16 at a time on one workspace of cfh_path_ws_bytes(M, ...) bytes
 * (the same size for every M >= 16). */
int64_t cfh_path_ws_bytes(int M, int d, int ffn_mult, int order);
int cfh_path_residual(const void* const* ph, int order, int ffn_mult, int d, const int32_t* lastp,
                      int M, int nlive, const void* embed_w, const void* pred, long long pred_ld,
                      int rows_per_pred, void* hsum, void* ws, void* stream);

/* Depth 0 of _beam_chains / _beam_tree (cf/vllm_plugin/flow_proposer.py:1208, 1221-1225, 1288-1291) in one
 * launch: lastp [B][W][order] = -1 except lastp[b][w][0] = known0[b] (every beam of a chain, beam 0
 * of a tree), cum [B][W] = 0 for beam 0 and -inf for the others (chain; tree: 0 everywhere),
 * prev_ids [B][W] = -1 (tree; null for a chain).  known0: int64 [B] committed tokens. */
int cfh_beam_init(const int64_t* known0, int32_t* lastp, float* cum, int32_t* prev_ids, int B, int W,
                  int order, int tree, void* stream);

/* One depth of _beam_chains (cf/vllm_plugin/flow_proposer.py:1250-1259) for B chains of width W
 * (W*W <= 64): from the per-beam top-W rows vals/ids [B*W][W] (log-probs, shortlist-local ids),
 * cand = cum[b][w] + vals; (cum, flat) = top-W(cand) (ties to the lower flat index);
 * toks[b][w] = sl[ids[src][flat % W]] (global id), bps[b][w] = src = flat / W;
 * lastp[b][w] = [toks, lastp[b][src][0..order-2]].  cum [B][W] and lastp [B][W][order] in place. */
int cfh_beam_chain_step(const float* vals, const int32_t* ids, float* cum, int32_t* lastp,
                        const int32_t* sl, int32_t* toks, int32_t* bps, int B, int W, int order,
                        void* stream);

/* cfh_head_topk_packed with k = W over the M = B W beam rows, then cfh_beam_chain_step on them (sl:
 * the ids' map, as there): the merge of the head's candidate lists and the beam step run as one
 * launch, a workgroup a chain, a wave a beam row, then the step on the chain's rows.  vals / ids /
 * lse are written as cfh_head_topk_packed writes them and cum / lastp / toks / bps as
 * cfh_beam_chain_step does; same results as the two calls.  One depth of _beam_chains' _head +
 * _bias + top-k + chain step (cf/vllm_plugin/flow_proposer.py:1234-1259). */
int cfh_head_topk_packed_beam_chain(const void* h, int M, int d, const void* packed, int n, const void* a,
                                    const int32_t* a_ids, int a_ids_stride, int r, float* vals, int32_t* ids,
                                    float* lse, void* ws, float* cum, int32_t* lastp, const int32_t* sl,
                                    int32_t* toks, int32_t* bps, int B, int W, int order, void* stream);

/* One depth of _beam_tree (:1300-1330): F live frontier slots, topb children each, keep the best
 * k = min(keep, F*topb); writes node tokens to out[b][base + i] and parent node indices to
 * out[b][ld_out/2 + base + i]; cum/lastp/prev_ids are [B][keep](...) frontier arrays, updated. */
int cfh_beam_tree_step(const float* vals, const int32_t* ids, float* cum, int32_t* lastp,
                       int32_t* prev_ids, const int32_t* sl, int32_t* out, int ld_out, int base,
                       int B, int F, int topb, int keep, int order, void* stream);

/* Backtrack of _beam_chains (:1261-1267): idx = first arg-max of cum [B][W]; for each depth s from
 * the last, out[b][s] = toks[s][b][idx], idx = bps[s][b][idx].  toks/bps [K][B][W]. */
int cfh_beam_backtrack(const float* cum, const int32_t* toks, const int32_t* bps, int B, int W, int K,
                       int64_t* out, void* stream);

/* ---------------------------------------------------------------- tree gated delta net
 * tree_gated_delta_scan (cf/kernels/tree_scan.py:41-73): per node n (BFS order, parent[n] < n,
 * -1 = root reading S0): S = exp(g) S_parent; delta = (v - S^T k) beta; S += k (x) delta;
 * out = S^T q, with q,k l2-normalised (l2mode 0: x/(|x|+1e-6), 1: x/sqrt(|x|^2+1e-6)) and
 * q scaled by Dk^-1/2.
 *   q,k [N][H][Dk] bf16, v [N][H][Dv] bf16, g,beta [N][H] fp32, S0 [H][Dk][Dv] fp32,
 *   out [N][H][Dv] fp32, states [N][H][Dk][Dv] fp32 or NULL.  Dk == 128, Dv % 64 == 0, N <= 256.
 * Replaces the fork's gdn_verify (patch:4606-4660) / tree_ssm Triton kernels for this layout. */
int cfh_gdn_tree(const void* q, const void* k, const void* v, const float* g, const float* beta,
                 const float* S0, const int32_t* parent, int N, int H, int Dk, int Dv,
                 int use_l2norm, int l2mode, float* out, float* states, void* stream);

/* The serving (vLLM) form of the tree GDN (cf/vllm_tree/tree_ssm.py:256-311, path-parallel;
 * bit-identical by construction to the per-node slot form :34-77 that stores each node's state and
 * has its children read it back):
 *   mixed_qkv [N][2 H K + HV V] bf16 (q heads | k heads | HV value heads; value head hv uses q/k
 *   head hv / (HV / H)); a, b [N][HV] bf16; A_log, dt_bias [HV] fp32;
 *   g = -exp(A_log) softplus(a + dt_bias) (softplus = identity above 20), beta = bf16(sigmoid(b));
 *   q, k l2-normalised as x / sqrt(|x|^2 + 1e-6) (use_l2norm), q scaled by `scale`;
 *   ssm_state [slots][HV][V][K], bf16 (state_bf16 = 1) or fp32: every node starts from slot
 *   prefix_slot, replays its root->node path with each ancestor's state rounded to the storage
 *   type, writes its state to slot node_slots[n] and o [N][HV][V] bf16.
 * parent [N] int32 (BFS order, -1 = root).  K == 128, V % 64 == 0, N <= 256; ssm_state holds
 * nslots slots and 0 <= prefix_slot < nslots.  Node slots are validated on the device, so the call
 * never synchronises and can be captured: a node whose slot lies outside [0, nslots), equals
 * prefix_slot or is shared with another node gets NaN outputs, writes no slot, and sets status[0]
 * to 1 (status: one int32 the caller zeroes, or NULL).  Replaces tree_scan_gdn_recurrence[_path]. */
int cfh_gdn_tree_vllm(const void* mixed_qkv, const void* a, const void* b, const float* A_log,
                      const float* dt_bias, void* ssm_state, int state_bf16, int nslots,
                      const int32_t* node_slots, const int32_t* parent, int prefix_slot, int N, int H,
                      int HV, int K, int V, int use_l2norm, float scale, void* out, int32_t* status,
                      void* stream);

/* ---------------------------------------------------------------- rest of the tree verify
 * Tree causal conv1d, width 4 (cf/vllm_tree/tree_ssm.py:393-438; depth form :189-253): node n
 * (BFS order, parent [N] node index, -1 = root) sees the last three inputs of its root->node path,
 * the prefix slot's state before the root; out = act(bias + bf16(s0 w0) + bf16(s1 w1) +
 * bf16(s2 w2) + bf16(x w3)) with fp32 accumulation left to right, act = SiLU (silu = 1) or none;
 * the node's state (s1, s2, x, s3) goes to slot node_slots[n].  x [N][x_ld], out [N][out_ld],
 * conv_state [slots][dim][4], weight [dim][4], bias [dim] (or NULL): all bf16. */
int cfh_tree_conv(const void* x, int x_ld, void* conv_state, const void* weight, const void* bias,
                  const int32_t* node_slots, const int32_t* parent, int prefix_slot, int N, int dim, int silu,
                  void* out, int out_ld, void* stream);

/* The draft-tree rows' ancestor-masked attention merged with the shared-prefix half
 * (_tree_suffix_eager + merge_attn_states, patch lines 529-575; fused form tree_attn_fused.cu):
 * per request s, node n, head h: softmax over the nodes m with not_anc[s][n][m] == 0 of
 * scale * q[idx[s][n]][h] . k[idx[s][m]][h / (H/Hkv)] (fp32), P.V in fp32 rounded to the element
 * type, lse_s = max + log(sum); then merged with prefix_out [S*N][H][D] / prefix_lse [H][S*N]
 * (fp32) by the log-sum-exp rule and written to out[idx[s][n]][h].  q/k/v/out rows are [.][heads][D]
 * with row strides q_ld/k_ld/v_ld/o_ld (elements); bf16 (is_bf16) or fp16; D in {64, 128, 256};
 * N <= 128; pointers and strides aligned to D/32 bytes (each lane reads D/64 elements at once). */
int cfh_tree_attn_merge(const void* q, int q_ld, const void* k, int k_ld, const void* v, int v_ld, void* out,
                        int o_ld, const void* prefix_out, const float* prefix_lse, const int32_t* idx,
                        const uint8_t* not_anc, float scale, int S, int N, int H, int Hkv, int D, int is_bf16,
                        void* stream);

/* Greedy tree verify (tree_rejection_sample + tree_greedy_descent_kernel, patch lines 433-550):
 * row_argmax[r] = first arg-max of logits row r (n_rows rows of V, row stride ld, bf16 or fp16);
 * then per request b (its rows s0 = cu_sampled[b] - n - 1 .. with n = its draft count from
 * cu_draft, inclusive cumulative counts): from the root row, emit the target's token, step to the
 * first child (parents: local parent, -1 = root) whose draft token equals it, repeat.
 * out_tokens [B][max_spec+1] (accepted drafts + the bonus, -1 padded), accepted_path
 * [B][max_spec] (node per depth, -1 padded), accepted_len [B]; row_argmax [n_rows] receives the
 * arg-max of every row of the B requests; ws: cfh_tree_accept_ws_bytes(n_rows) bytes. */
int64_t cfh_tree_accept_ws_bytes(int n_rows);
int cfh_tree_greedy_accept(const void* logits, long long ld, int V, int n_rows, int is_bf16, const int32_t* cu_draft,
                           const int32_t* cu_sampled, const int32_t* draft_ids, const int32_t* parents, int B,
                           int max_spec, int32_t* out_tokens, int32_t* accepted_path, int32_t* accepted_len,
                           int32_t* row_argmax, void* ws, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CFHIP_H */
