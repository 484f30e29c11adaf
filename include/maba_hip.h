/*
 * maba_hip.h -- C ABI of the MI355X (gfx950) HIP backend for the Maba v2 hot path.
 *
 * Every entry point takes plain tensor descriptors (device pointer, dtype code,
 * shape and element strides), scalar parameters and a hipStream_t passed as
 * void*.  No entry point allocates persistent device memory; the ones that need
 * scratch take a caller-provided workspace and have a *_workspace_size query.
 * All work is enqueued on the given stream; nothing synchronises the host.
 *
 * Return value: 0 on success, MABA_ERR_* otherwise; the message of the last
 * failure on the calling thread is returned by maba_hip_last_error().
 *
 * Reference interfaces replaced (paths relative to the reference checkout):
 *   maba_hip_dgda_prefill           maba_sparse/kernels/dispatcher.py:258-327
 *                                   (op "dgda_prefill"; math common.py:229-268)
 *   maba_hip_dgda_step              dispatcher.py:330-396
 *                                   (op "dgda_step"; math common.py:271-309)
 *   maba_hip_compute_centroids      dispatcher.py:399-421
 *                                   (op "compute_centroids"; common.py:329-350)
 *   maba_hip_index_topk             dispatcher.py:424-465
 *                                   (op "index_topk"; cpu_indexer.py:53-112)
 *   maba_hip_index_topk_decode      layers/indexer.py:101-112 (inline decode
 *                                   scoring + torch.topk; no dispatcher op)
 *   maba_hip_stream_superposition   dispatcher.py:468-508
 *                                   (op "stream_superposition"; common.py:406-438)
 *   maba_hip_hca_pool               layers/sparse_attention.py:206 (block means
 *                                   of the latent cache for the HCA stream)
 *   maba_hip_maba_sa_decode         layers/sparse_attention.py:79-219,263-275
 *                                   (local + sparse + HCA decode streams and the
 *                                   gate superposition; inline torch code in the
 *                                   reference, no dispatcher op)
 *   maba_hip_maba_sa_prefill        layers/sparse_attention.py:95-105,145-171,
 *                                   173-219,275 (the three prefill streams over
 *                                   dense masks and the gate; inline torch code)
 *   maba_hip_maba_sa_prefill_latent the same streams over the latent cache with the
 *                                   absorbed projections
 *   maba_hip_dgda_prologue          layers/dgda.py:103-121,186-207 (the DGDA
 *                                   layer's conv + SiLU with carried history,
 *                                   gate activations and key normalisation;
 *                                   inline torch code in the reference)
 *   maba_hip_dgda_layer_prefill     layers/dgda.py:103-121,186-233 (the prologue
 *                                   above fused into the prefill kernels' input
 *                                   staging, then the chunked recurrence)
 *   maba_hip_dgda_layer_step        layers/dgda.py:103-121,186-207 then
 *                                   dispatcher.py:330-396 (the decode prologue above
 *                                   and the step in one launch)
 *   maba_hip_cache_append           layers/indexer.py:62-82 (key cache, complete
 *                                   and tail centroids), layers/sparse_attention.py:
 *                                   206, 241-251 (latent rows, HCA block means)
 *   maba_hip_index_topk_decode_dev  layers/indexer.py:101-112 with the centroid
 *                                   count read from device memory
 *   maba_hip_maba_sa_decode_dev     layers/sparse_attention.py:79-219,263-275 with
 *                                   the sequence length read from device memory
 *   maba_hip_cache_append_heads     maba_hip_cache_append plus the token's absorbed
 *                                   queries W_k,h^T q_h and gate logits W_g x + b
 *                                   (layers/sparse_attention.py:79-219, 274)
 *   maba_hip_maba_sa_decode_dev_heads  maba_hip_maba_sa_decode_dev plus the value
 *                                   up-projection W_v,h z_h of each head
 *                                   (layers/sparse_attention.py:208, absorbed)
 *   maba_hip_rmsnorm                model.py:11-22 (RMSNorm) and the gated residual
 *                                   of MabaBlock, model.py:92-128
 *   maba_hip_swiglu                 model.py:25-38 (SwiGLU activation)
 *   maba_hip_argmax_rows            model.py:279-313 (the greedy pick, torch.argmax)
 *   maba_hip_decode_linear          nn.Linear of one decode token per sequence
 *                                   (model.py:25-38, 92-128, the layers' projections),
 *                                   its input from RMSNorm, the gated residual +
 *                                   RMSNorm or SwiGLU (model.py:11-38, 92-128) in the
 *                                   same launch
 */
#ifndef MABA_HIP_H
#define MABA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum maba_dtype {
  MABA_F32 = 0,
  MABA_F16 = 1,
  MABA_BF16 = 2,
  MABA_F64 = 3,
  MABA_I64 = 4,
  MABA_I32 = 5
};

enum maba_status {
  MABA_OK = 0,
  MABA_ERR_INVALID = 1,     /* bad shape / argument (Python: ValueError) */
  MABA_ERR_DTYPE = 2,       /* unsupported dtype (Python: TypeError) */
  MABA_ERR_UNSUPPORTED = 3, /* valid but not implemented here (Python: NotImplementedError) */
  MABA_ERR_HIP = 4,         /* HIP runtime error (Python: RuntimeError) */
  MABA_ERR_WORKSPACE = 5    /* workspace too small (Python: RuntimeError) */
};

/* A strided view of device memory.  Unused trailing dims have shape 1. */
typedef struct maba_tensor {
  void* data;
  int32_t dtype;
  int32_t ndim;
  int64_t shape[4];
  int64_t stride[4]; /* in elements */
} maba_tensor;

const char* maba_hip_last_error(void);
int maba_hip_abi_version(void);

/*
 * DGDA chunked prefill.  q,k,alpha,log_alpha,b: [B,H,L,dk]; v,w: [B,H,L,dv];
 * initial_state: [B,H,dk,dv] or NULL (zeros).  alpha or log_alpha may be NULL
 * (not both); log_alpha wins when both are given.  Any of the gates may be a
 * stride-0 broadcast along the channel axis.  out: [B,H,L,dv],
 * final_state: [B,H,dk,dv]; dtypes f32/f16/bf16 independently per tensor.
 * chunk_size is accepted for signature parity; the result does not depend on it.
 * dk, dv in {32, 64, 128} with q, k, v of one dtype and the gates fp32 (or in q's
 * 16-bit dtype) take the sequence-parallel MFMA paths, which need the workspace the
 * size query returns (it depends on the current device's compute-unit count); every
 * other shape up to 128 runs a sequential kernel and needs none (the query returns 0).
 */
size_t maba_hip_dgda_prefill_workspace_size(const maba_tensor* q, const maba_tensor* v,
                                            const maba_tensor* log_alpha_or_alpha,
                                            const maba_tensor* b);
int maba_hip_dgda_prefill(const maba_tensor* q, const maba_tensor* k, const maba_tensor* v,
                          const maba_tensor* alpha, const maba_tensor* log_alpha,
                          const maba_tensor* b, const maba_tensor* w,
                          const maba_tensor* initial_state, maba_tensor* out,
                          maba_tensor* final_state, int chunk_size, void* workspace,
                          size_t workspace_bytes, void* stream);

/* DGDA single decode step.  q,k,alpha,log_alpha,b: [B,H,dk]; v,w: [B,H,dv];
 * state / new_state: [B,H,dk,dv] (state NULL = zeros); out: [B,H,dv].  new_state may be
 * state itself (the state is updated in place).  dk, dv in {32, 64, 128}, fp32 gates, q, k,
 * v of one dtype and an fp32 or bf16 state with unit column stride (rows dv apart unless
 * dk = dv = 64) take the four-wave kernel; other shapes a generic one. */
int maba_hip_dgda_step(const maba_tensor* q, const maba_tensor* k, const maba_tensor* v,
                       const maba_tensor* alpha, const maba_tensor* log_alpha,
                       const maba_tensor* b, const maba_tensor* w, const maba_tensor* state,
                       maba_tensor* out, maba_tensor* new_state, void* stream);

/* Block centroids 0.5*(mean+max) over block_size tokens, zero-padded tail.
 * k_idx: [B,L,d]; out: [B,ceil(L/block_size),d] (same dtype as k_idx). */
int maba_hip_compute_centroids(const maba_tensor* k_idx, maba_tensor* out, int block_size,
                               void* stream);

/* Causal prefill scoring + top-k.  q_idx: [B,L,d]; centroids: [B,nb,d];
 * out_idx: int64 [B,L,min(top_k,nb)]; out_scores: [B,L,nb] or NULL.  Any top_k; above 64 the
 * rows are sorted whole (at most 16384 blocks, MABA_ERR_UNSUPPORTED beyond). */
int maba_hip_index_topk(const maba_tensor* q_idx, const maba_tensor* centroids,
                        float lambda_dist, int top_k, int block_size, maba_tensor* out_idx,
                        maba_tensor* out_scores, void* stream);

/* Decode scoring (query block = nb-1, no mask) + top-k for Hq query heads
 * sharing one centroid set.  q: [B,Hq,d]; centroids: [B,nb,d];
 * out_idx: int64 [B,Hq,min(top_k,nb)]; out_scores: f32 [B,Hq,nb] or NULL.  Any top_k; above 64
 * the rows are sorted whole (at most 16384 blocks, MABA_ERR_UNSUPPORTED beyond; no workspace). */
size_t maba_hip_index_topk_decode_workspace_size(int64_t B, int64_t Hq, int64_t nb, int top_k);
int maba_hip_index_topk_decode(const maba_tensor* q, const maba_tensor* centroids,
                               float lambda_dist, int top_k, maba_tensor* out_idx,
                               maba_tensor* out_scores, void* workspace,
                               size_t workspace_bytes, void* stream);

/* out = g0*o_local + g1*o_sparse + g2*o_hca; o_*: [B,H,L,D]; gate: [B,L,3] or
 * [B,H,L,3] logits (softmax taken) or weights (is_weights != 0). */
int maba_hip_stream_superposition(const maba_tensor* o_local, const maba_tensor* o_sparse,
                                  const maba_tensor* o_hca, const maba_tensor* gate,
                                  int is_weights, maba_tensor* out, void* stream);

/* Means of complete pool-token blocks of a latent cache: c_kv [B,L,dc] ->
 * out [B,L/pool,dc] (rounded to out's dtype). */
int maba_hip_hca_pool(const maba_tensor* c_kv, maba_tensor* out, int pool, void* stream);

/*
 * Fused MABA-SA decode step over an MLA latent cache (latent absorption):
 *   q_lat     [B,H,dc]  per-head query already mapped into latent space
 *                       (W_k,h^T q_h, scale applied by the kernel)
 *   c_kv      [B,Lmax,dc] latent cache, first L rows valid
 *   hca       [B,>=L/pool,dc] means of complete pool-blocks
 *   idx       int64 [B,Hi,K] selected blocks, Hi in {1,H}
 *   gate      [B,3] or [B,H,3] gate logits
 *   out_lat   f32 [B,H,dc]  sum_s g_s * sum_j p_sj c_j  (latent-space output;
 *                       the caller applies W_v,h).  When L < pool the HCA
 *                       stream is the running mean of c[0..L-1]
 *                       (sparse_attention.py:189-199), computed in-kernel.
 * scale = 1/sqrt(d_head) is passed explicitly.
 */
size_t maba_hip_maba_sa_decode_workspace_size(int64_t B, int64_t H, int64_t dc, int64_t L,
                                              int64_t K, int window, int n_sink, int pool);
int maba_hip_maba_sa_decode(const maba_tensor* q_lat, const maba_tensor* c_kv,
                            const maba_tensor* hca, const maba_tensor* idx,
                            const maba_tensor* gate, int64_t L, float scale, int window,
                            int n_sink, int block_size, int pool, maba_tensor* out_lat,
                            void* workspace, size_t workspace_bytes, void* stream);

/*
 * maba_hip_maba_sa_decode without a workspace argument: no counterpart in the reference.
 * For callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same arguments, checks and result as
 * maba_hip_maba_sa_decode; the partial slots live in a static device array of
 * MABA_SA_STATIC_SCRATCH_BYTES per GPU (held until the process ends), whose address is
 * queried once per device on the first call with that device current.  A call whose
 * partials need more (maba_hip_maba_sa_decode_workspace_size bounds it) fails with
 * MABA_ERR_WORKSPACE before launching anything.  Calls allocate nothing.  Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (different streams or
 * threads) race and must be serialised by the caller.  Nothing in the array needs to
 * start at zero: each call writes every slot it reads.
 */
#define MABA_SA_STATIC_SCRATCH_BYTES ((size_t)8 << 20)
int maba_hip_maba_sa_decode_static(const maba_tensor* q_lat, const maba_tensor* c_kv,
                                   const maba_tensor* hca, const maba_tensor* idx,
                                   const maba_tensor* gate, int64_t L, float scale, int window,
                                   int n_sink, int block_size, int pool, maba_tensor* out_lat,
                                   void* stream);

/*
 * MABA-SA prefill: every query's local, sparse and HCA streams and their gate.
 *   q [B,H,Lq,dh], k, v [B,H,Lkv,dh] (bf16, unit channel stride, 16-byte aligned rows,
 *   dh in {32,64,128}); query t sits at position pos = Lkv - Lq + t.
 *   kh, vh [B,H,Lkv/pool,dh] bf16: keys / values of the complete-block means (NULL when
 *   Lkv < pool).  early [B,H,n_early,dh]: the HCA rows of the queries with pos < pool-1
 *   (n_early of them; NULL when none).  idx int64 [B,Lq|1,K], K <= 64: each query's
 *   64-token blocks (block_size must be 64; a block listed twice counts twice).
 *   gate [B,Lq,3] or [B,H,Lq,3] logits.  out [B,H,Lq,dh] f32 or bf16.
 *   local: keys j <= pos with pos - j < window or j < min(n_sink, Lkv); sparse: the listed
 *   blocks' tokens <= pos; HCA: means e with (e+1)*pool - 1 <= pos.  Lkv <= 1,048,576.
 */
int maba_hip_maba_sa_prefill(const maba_tensor* q, const maba_tensor* k, const maba_tensor* v,
                             const maba_tensor* kh, const maba_tensor* vh, const maba_tensor* early,
                             const maba_tensor* idx, const maba_tensor* gate, float scale,
                             int window, int n_sink, int block_size, int pool, maba_tensor* out,
                             void* stream);

/*
 * MABA-SA prefill in latent form (the same streams and gate as maba_hip_maba_sa_prefill,
 * layers/sparse_attention.py:95-105,145-171,173-219,275): query t of q_lat [B,Lq,H,dc]
 * (W_k,h^T q_h; f32/bf16) sits at position Lkv - Lq + t of the bf16 latent cache
 * c_kv [B,Lkv,dc] (16-byte aligned rows, dc a multiple of 32 up to 128, H <= 16) and attends,
 * per head, to the local window + sinks, the tokens <= pos of its blocks idx [B,Lq|1,K]
 * (int64, K <= 64, block_size <= 64, a block listed twice counts twice), and the complete means of
 * hca [B,>=Lkv/pool,dc] (bf16) with (e+1) pool - 1 <= pos, or the running mean of c[0..pos]
 * before pool - 1; gate [B,Lq,3] or [B,H,Lq,3] logits.  out_lat f32 [B,Lq,H,dc] (unit
 * channel stride) = sum_s g_s z_s; the caller applies W_v,h.  A stream without a valid key
 * contributes zero.
 */
int maba_hip_maba_sa_prefill_latent(const maba_tensor* q_lat, const maba_tensor* c_kv,
                                    const maba_tensor* hca, const maba_tensor* idx,
                                    const maba_tensor* gate, float scale, int window, int n_sink,
                                    int block_size, int pool, maba_tensor* out_lat, void* stream);

/*
 * DGDA layer prologue.  xs[0..5]: the q, k, v, alpha, erase and write projections
 * [B,L,C] (C = 64*H, H <= 16; f32 or bf16, one dtype, unit channel stride).
 * conv_w[0..2]: depthwise kernels [C,1,4] of q, k, v.  hist: NULL (zeros) or three
 * [B,C,3] carried conv inputs, oldest first.  Outputs ys[0..6] [B,L,C]:
 *   q = silu(conv_q([hist, x_q])), k = silu(conv_k(...)) / (||.||_head + eps),
 *   v = silu(conv_v(...))                        (f32 or bf16, one dtype)
 *   log_alpha = max(-softplus(x_alpha), -14), alpha = exp(log_alpha) (ys[4] may be
 *   NULL), b = sigmoid(x_erase), w = sigmoid(x_write)    (f32 or bf16, one dtype)
 * new_hist[0..2] [B,C,3]: the last three conv inputs of q, k, v; must not alias hist
 * unless L == 1 (a single token reads each channel's history before writing it).
 */
int maba_hip_dgda_prologue(const maba_tensor* const* xs, const maba_tensor* const* conv_w,
                           const maba_tensor* const* hist, float eps, maba_tensor* const* ys,
                           maba_tensor* const* new_hist, void* stream);

/*
 * DGDA layer prefill with the prologue fused into the recurrence kernels' input staging:
 * q, k, v, the gates and the key norm are formed in fp32 inside the kernels and never
 * stored.  xs: the six bf16 projections [B,L,C] (q, k, v, decay, erase, write; unit channel
 * stride, 8-byte aligned rows, C = 64 H), conv_w [C,1,4] x3 (f32/bf16), hist [B,C,3] x3 bf16
 * or NULL (zeros), eps the key-norm epsilon, initial_state [B,H,64,64] or NULL, out
 * [B,H,L,64] (f32/bf16, unit channel stride; a [B,L,C] buffer viewed head-major), final_state
 * [B,H,64,64], new_hist [B,C,3] x3 (f32/bf16; may alias hist: it is written last).  L >= 1.
 * The workspace is sized by maba_hip_dgda_layer_prefill_workspace_size(B, H, L).
 */
size_t maba_hip_dgda_layer_prefill_workspace_size(int64_t B, int64_t H, int64_t L);
int maba_hip_dgda_layer_prefill(const maba_tensor* const* xs, const maba_tensor* const* conv_w,
                                const maba_tensor* const* hist, float eps, const maba_tensor* initial_state,
                                maba_tensor* out, maba_tensor* final_state, maba_tensor* const* new_hist,
                                void* workspace, size_t workspace_bytes, void* stream);

/*
 * Serving path: a decode step whose position lives in device memory, so that one captured
 * HIP graph serves every position.  `pos` / `d_len` are device pointers to one int64.
 *
 * Cache append (one launch per decode token and MABA-SA layer).  Writes c_new [B,dc] to row
 * p = *pos of c_cache [B,Lmax,dc] and k_new [B,di] to row p of k_cache [B,Lmax,di]; when row
 * p completes a pool-block, hca[b, (p+1)/pool - 1] = the block's mean; and
 * centroids[b, p/block_size] = 0.5 (mean + max) of the block holding row p, zero-padded when
 * incomplete (the padding counts in the mean and the max).  All bf16, unit channel strides;
 * hca [B,>=Lmax/pool,dc], centroids [B,>=ceil(Lmax/block_size),di].  The caller advances *pos.
 */
int maba_hip_cache_append(const maba_tensor* c_new, const maba_tensor* k_new, const int64_t* pos,
                          maba_tensor* c_cache, maba_tensor* k_cache, maba_tensor* hca,
                          maba_tensor* centroids, int pool, int block_size, void* stream);

/* maba_hip_cache_append, and in the same launch the token's absorbed queries and gate logits:
 * q_lat [B,H,dc] f32 (unit channel stride) = W_k,h^T q_h for q_heads [B,H*dh] and
 * w_k [H*dh,dc] (unit column stride), summed in fp32; gate_out [B,3] = bf16(gate_in + gate_bias)
 * for gate_in [B,3], gate_bias [3].  All bf16 but q_lat. */
int maba_hip_cache_append_heads(const maba_tensor* c_new, const maba_tensor* k_new, const int64_t* pos,
                                maba_tensor* c_cache, maba_tensor* k_cache, maba_tensor* hca,
                                maba_tensor* centroids, int pool, int block_size,
                                const maba_tensor* q_heads, const maba_tensor* w_k,
                                const maba_tensor* gate_in, const maba_tensor* gate_bias,
                                maba_tensor* q_lat, maba_tensor* gate_out, void* stream);

/* maba_hip_index_topk_decode over the first nb = ceil(*d_len / block_size) rows of centroids
 * [B,Ncap,d] (bf16 MFMA path; nb must reach top_k).  out_idx int64 [B,Hq,top_k]; workspace
 * sized by maba_hip_index_topk_decode_workspace_size(B, Hq, Ncap, top_k). */
int maba_hip_index_topk_decode_dev(const maba_tensor* q, const maba_tensor* centroids,
                                   const int64_t* d_len, int block_size, float lambda_dist,
                                   int top_k, maba_tensor* out_idx, void* workspace,
                                   size_t workspace_bytes, void* stream);

/* maba_hip_maba_sa_decode with L = *d_len <= L_cap (bf16 MFMA path); workspace sized by
 * maba_hip_maba_sa_decode_workspace_size(..., L_cap, ...). */
int maba_hip_maba_sa_decode_dev(const maba_tensor* q_lat, const maba_tensor* c_kv,
                                const maba_tensor* hca, const maba_tensor* idx,
                                const maba_tensor* gate, const int64_t* d_len, int64_t L_cap,
                                float scale, int window, int n_sink, int block_size, int pool,
                                maba_tensor* out_lat, void* workspace, size_t workspace_bytes,
                                void* stream);

/* maba_hip_maba_sa_decode_dev, and in its merge launch the value up-projection of each head:
 * out_heads [B,H*dh] bf16 = bf16(W_v,h z_h) for w_v [H*dh,dc] bf16 (dh <= 64, unit column
 * stride, 8-byte aligned rows), summed in fp32; out_lat still receives z. */
int maba_hip_maba_sa_decode_dev_heads(const maba_tensor* q_lat, const maba_tensor* c_kv,
                                      const maba_tensor* hca, const maba_tensor* idx,
                                      const maba_tensor* gate, const int64_t* d_len, int64_t L_cap,
                                      float scale, int window, int n_sink, int block_size, int pool,
                                      const maba_tensor* w_v, maba_tensor* out_heads,
                                      maba_tensor* out_lat, void* workspace, size_t workspace_bytes,
                                      void* stream);

/* One decode token of the DGDA layer after its input projection: the single-token prologue
 * of maba_hip_dgda_prologue (conv + SiLU over the carried history, key norm, gates, new
 * history) and maba_hip_dgda_step in one launch, with q, k, v rounded to bf16 and the gates
 * kept in fp32 as those two store them (the results equal theirs).  xs: the six bf16
 * projections [B,C] or [B,1,C] (q, k, v, decay, erase, write; unit channel stride, C = 64 H),
 * conv_w [C,1,4] x3 (f32/bf16, one dtype), hist [B,C,3] x3 bf16 (all three) or NULL (zeros), eps the
 * key-norm epsilon, state [B,H,64,64] f32/bf16 or NULL (zero), out [B,H,64] f32/bf16,
 * new_state like state (may alias it), new_hist [B,C,3] x3 bf16 (may alias hist). */
int maba_hip_dgda_layer_step(const maba_tensor* const* xs, const maba_tensor* const* conv_w,
                             const maba_tensor* const* hist, float eps, const maba_tensor* state,
                             maba_tensor* out, maba_tensor* new_state, maba_tensor* const* new_hist,
                             void* stream);

/* h = x' / sqrt(mean(x'^2) + eps) * weight over the last dim C (even, <= 2048), where
 * x' = x + gate * mo when mo is given (gate [C]), else x; x' is written to x_out when given
 * (may alias x).  x, mo, x_out, h: [..,C] f32 or bf16 rows; weight, gate f32 or bf16. */
int maba_hip_rmsnorm(const maba_tensor* x, const maba_tensor* mo, const maba_tensor* gate,
                     const maba_tensor* weight, float eps, maba_tensor* x_out, maba_tensor* h,
                     void* stream);

/* out [..,I] = silu(g) * u for gate_up [..,2I] = [g | u] (f32 or bf16, one dtype). */
int maba_hip_swiglu(const maba_tensor* gate_up, maba_tensor* out, void* stream);

/* y = A weight^T for a few rows (one decode token per sequence), bf16 with fp32 accumulation.
 * weight [N,K] bf16 (unit K stride, 16-byte aligned rows, K a multiple of 32, K <= 4096).
 * A is built in the same launch from a ([M,K] or [M,1,K] bf16 rows, 16-byte aligned):
 *   act 0, norm_w NULL:       A = a
 *   rows [M] or [M,1] int64:  A[m] = a[rows[m]] for a table a [V,K] (rows clamped into [0, V))
 *   act 0, norm_w [K]:        A = bf16(a / sqrt(mean(a^2) + eps) * norm_w)          (K <= 2048)
 *   act 0, norm_w, mo, gate:  x' = bf16(a + gate * mo) is written to x_out and A is the RMSNorm of
 *                             x' as above; x_out may overlap neither a nor mo     (K <= 2048)
 *   act 1:                    A = bf16(silu(a[:, :K]) * a[:, K:2K]) for a [M,2K]
 * y [M,N] or [M,1,N] bf16, unit column stride, overlapping no input. */
int maba_hip_decode_linear(const maba_tensor* a, const maba_tensor* rows, const maba_tensor* mo,
                           const maba_tensor* gate, const maba_tensor* norm_w, float eps, int act,
                           const maba_tensor* weight, maba_tensor* x_out, maba_tensor* y, void* stream);

/* out[m] = the index of the first maximum of row m of x ([M,V] or [M,1,V], bf16 or f32, unit
 * column stride, 16-byte aligned rows, V a multiple of 8 (bf16) or 4 (f32)), as torch.argmax:
 * NaN counts as the maximum and -0 equals +0.  out int64 [M] or [M,1]. */
int maba_hip_argmax_rows(const maba_tensor* x, maba_tensor* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MABA_HIP_H */
