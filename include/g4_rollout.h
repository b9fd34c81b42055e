/*
 * g4_rollout.h — C ABI of libg4rollout.so, the MI355X (gfx950) kernels behind the Gemma 4
 * rollout prefill + KV-cache decode path of gemma4_posttrain_jax.
 *
 * The reference has no native layer: each entry point below replaces an XLA-lowered JAX
 * expression of gemma4_posttrain_jax/model.py, cited per function. All entry points are
 * stream-ordered on the `hipStream_t` passed as `stream`, launch nothing else, allocate
 * nothing, never synchronise the device, and keep no state between calls (reentrant). The one
 * piece of library state is the per-device set-up of g4_init, done once per device and guarded
 * against concurrent first calls. They return 0 on success or a negative G4_ERR_* code after a
 * host-side argument check, before any launch; `g4_last_error()` then describes the failure
 * (thread-local text).
 *
 * Device data layout (per cache layer, element type = `dtype`):
 *   cache_k   [B, Hkv, slot_stride/32, D/KR, 2, 16, KR], KR = min(D, 32): each 32-slot chunk in
 *             the order of the attention MFMA's A operand; key (b,h,slot,d), r = slot%32, at
 *             (b*Hkv + h)*slot_stride*D + ((((slot/32)*(D/KR) + d/KR)*2 + (r/4)%2)*16
 *             + 4*(r/8) + r%4)*KR + d%KR, so one 16-lane x 32-dim operand load reads one
 *             contiguous 1 KiB block (bf16)
 *   cache_vt  [B, Hkv, slot_stride/8, D, 8]   values in groups of 8 slots, each group d-major;
 *             value (b,h,slot,d) at ((b*Hkv + h)*slot_stride + (slot/8)*8)*D + d*8 + slot%8,
 *             so the 8 slots of one value dim are contiguous (one 16-byte MFMA operand in bf16)
 *             and one slot's D values lie in one 8*D-element span (an append touches D/8
 *             cache lines of 128 bytes in bf16, not D)
 * `capacity` is the logical slot count: C (= prompt + new tokens) for a linear (global-layer)
 * cache, Wc = min(window, C) for a ring (sliding-layer) cache. `slot_stride` >= capacity is a
 * multiple of 64, so every K row and every value group starts 128-byte aligned.
 * Query/output rows of one kv head are contiguous: q and attention output are
 * [B, S, Hkv, R, D] (R = query heads per kv head; reference head order is h*R + r).
 * key_mask is [B, key_mask_stride] uint8 over absolute positions (1 = real token).
 */
#ifndef G4_ROLLOUT_H
#define G4_ROLLOUT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  G4_OK = 0,
  G4_ERR_INVALID = -1,     /* bad shape / null pointer / unsupported combination */
  G4_ERR_UNSUPPORTED = -2, /* valid but not implemented for this dtype / size */
  G4_ERR_LAUNCH = -3,      /* the HIP launch itself failed */
  G4_ERR_WORKSPACE = -4    /* workspace missing or too small */
};

/*
 * One-time set-up of the current HIP device: raises the dynamic-LDS limit of the decode and
 * prefill kernels that launch with more than the 64 KiB default (hipFuncSetAttribute). The first
 * call on a device does the work (std::call_once: concurrent first calls wait for it), later calls
 * return its recorded result. g4_decode_attention and g4_prefill_attention call it themselves
 * before their first launch on a device; a caller that captures those calls into a HIP graph calls
 * g4_init once per device beforehand, so that no set-up call falls inside the capture. No
 * reference counterpart: XLA sets kernel attributes when it compiles the module.
 */
int g4_init(void);

enum { G4_DTYPE_F32 = 0, G4_DTYPE_BF16 = 1 };
enum { G4_CACHE_LINEAR = 0, G4_CACHE_RING = 1 };

/* Flags of G4AppendArgs.flags. */
enum {
  G4_APPEND_NORM_K = 1, /* k = RMSNorm(k) * k_norm_weight (model.py:480) */
  G4_APPEND_NORM_V = 2, /* v = RMSNorm(v), no scale (model.py:482) */
  G4_APPEND_ROPE_K = 4, /* k = k*cos + rotate_half(k)*sin (model.py:481, 309-317) */
  G4_APPEND_NORM_Q = 8, /* q = RMSNorm(q) * q_norm_weight (model.py:465) */
  G4_APPEND_ROPE_Q = 16 /* q = RoPE(q) (model.py:466) */
};

/*
 * Fused q/k/v preparation + cache append. Replaces, for one layer:
 *   forward_rms_norm(q_norm) + forward_rotary_embedding on q   (model.py:465-466)
 *   forward_rms_norm(k_norm) + forward_rotary_embedding on k   (model.py:480-481)
 *   forward_rms_norm(None) on v                                 (model.py:482)
 *   _update_layer_cache(cache, k, v, start, circular)           (model.py:368-390)
 * Each of S new tokens of row b is written at absolute position p = write_pos[b] + s; a linear
 * cache stores it in slot p, a ring cache in slot p mod Wc, and of a chunk longer than Wc only
 * the last Wc tokens are stored (model.py:383-386). With flags == 0 and q == NULL this is the
 * pure data movement of _update_layer_cache and is bit-exact. With k == v == NULL only q is
 * prepared (kv-shared layers, model.py:469-470). RoPE tables are f32 [B, S, D]
 * (model.py:288-291); they are rounded to `dtype` before use, as model.py:313-314 does.
 */
typedef struct G4AppendArgs {
  int32_t dtype;        /* G4_DTYPE_*: inputs, cache and outputs */
  int32_t kind;         /* G4_CACHE_LINEAR or G4_CACHE_RING */
  int32_t batch;        /* B */
  int32_t seq;          /* S new tokens per row */
  int32_t kv_heads;     /* Hkv */
  int32_t group;        /* R = query heads per kv head (only read when q != NULL) */
  int32_t head_dim;     /* D: 64, 128, 256 or 512 */
  int32_t capacity;     /* logical slots: C (linear) or Wc (ring) */
  int32_t slot_stride;  /* physical slots per (b, h): >= capacity, multiple of 64 */
  int32_t flags;        /* G4_APPEND_* */
  float eps;            /* RMSNorm epsilon */
  int32_t write_pos_scalar;   /* start position used when write_pos == NULL (the reference's scalar length) */
  const int32_t* write_pos;   /* device [B] per-row start position, or NULL */
  const void* k;        /* token (b,s): k + (b*S + s)*in_row_stride, heads [Hkv, D] */
  const void* v;        /* same indexing as k (may alias k: K=V layers, model.py:479) */
  const void* q;        /* optional: token (b,s): q + (b*S + s)*in_row_stride, heads [Hkv, R, D] */
  int64_t in_row_stride;      /* elements between consecutive tokens of q / k / v */
  const void* q_norm_weight;  /* [D] in dtype (G4_APPEND_NORM_Q) */
  const void* k_norm_weight;  /* [D] in dtype (G4_APPEND_NORM_K) */
  const float* rope_cos;      /* [B, S, D] f32 (G4_APPEND_ROPE_*) */
  const float* rope_sin;      /* [B, S, D] f32 */
  void* cache_k;        /* key layout above: [B, Hkv, slot_stride/32, D/KR, 2, 16, KR] */
  void* cache_vt;       /* [B, Hkv, slot_stride/8, D, 8] (grouped values) */
  void* q_out;          /* optional [B, S, Hkv, R, D] prepared q */
  void* k_out;          /* optional prepared k of this chunk (prefill input), key layout with
                           slot_stride = chunk_stride */
  void* vt_out;         /* optional [B, Hkv, chunk_stride/8, D, 8] prepared v, grouped like cache_vt */
  int32_t chunk_stride; /* >= S, multiple of 64; required when k_out or vt_out is set */
} G4AppendArgs;

int g4_kv_append(const G4AppendArgs* args, void* stream);

/*
 * One-token GQA decode attention over a ring or linear cache. Replaces
 * make_cached_qk_masks (model.py:338-365) + the score/softmax/value einsums of
 * forward_attention (model.py:496-499) for S = 1, scale 1.0.
 * The query of row b sits at absolute position q_pos[b] (the cache length before this token's
 * append, i.e. the last written position). Validity of a key:
 *   linear slot t:  t <= q  and key_mask[b, t]
 *   ring slot r:    p = r + floor((q - r)/Wc)*Wc, p >= 0, p > q - window, key_mask[b, p]
 * Rounding follows the reference: scores rounded to `dtype`, masked scores = finfo(dtype).min,
 * f32 softmax over the whole row, probabilities rounded to `dtype`, f32-accumulated
 * probs @ v rounded to `dtype`. A row with no valid key averages all `capacity` slots, as the
 * reference's softmax over an all-min row does. Exact global softmax normalisation (not an
 * online rescale) keeps the probability rounding identical to the reference's.
 * With new_k/new_v set, the kernel first stores this token's K/V row (prepared, [B, Hkv, D])
 * at position q_pos[b] — the fused append — and attends over the updated cache.
 */
/*
 * Optional fused preparation for g4_decode_attention (the two-launch path only): instead of
 * prepared q / new_k / new_v, the raw projection rows, and the launch does g4_kv_append's work
 * itself -- q norm + RoPE, k norm + RoPE, the unscaled v norm (model.py:463-482) and the cache
 * append (model.py:368-390) -- with the same arithmetic. q_raw [B, Hkv, R, D], k_raw / v_raw
 * [B, Hkv, D] with in_row_stride elements between batch rows (the q/k/v projection output);
 * k_raw = NULL for a kv-shared layer (no append). rope_cos / rope_sin [B, D] f32 at the query
 * positions; flags as g4_kv_append's. Rows aligned to D/64 elements, cos / sin to 16 bytes.
 */
typedef struct G4DecodePrep {
  const void* q_raw;
  const void* k_raw;
  const void* v_raw;
  int64_t in_row_stride;
  const void* q_norm_weight;
  const void* k_norm_weight;
  const float* rope_cos;
  const float* rope_sin;
  float eps;
  int32_t flags;
} G4DecodePrep;

typedef struct G4DecodeArgs {
  int32_t dtype;
  int32_t kind;
  int32_t batch;
  int32_t kv_heads;
  int32_t group;        /* R <= 16 */
  int32_t head_dim;     /* bf16: 32, 64, 128, 256 or 512; f32: 8 .. 512 */
  int32_t capacity;     /* C or Wc */
  int32_t slot_stride;
  int32_t window;       /* sliding window W (ring caches); ignored for linear */
  int32_t q_pos_scalar; /* used when q_pos == NULL */
  const int32_t* q_pos; /* device [B] or NULL */
  const uint8_t* key_mask;     /* device [B, key_mask_stride] */
  int32_t key_mask_stride;     /* >= the largest absolute position + 1 (the full capacity C) */
  const void* q;        /* [B, Hkv, R, D] */
  const void* cache_k;  /* key layout above: [B, Hkv, slot_stride/32, D/KR, 2, 16, KR] */
  void* cache_vt;       /* [B, Hkv, slot_stride/8, D, 8]; written only with new_v */
  void* cache_k_w;      /* same as cache_k, writable; required with new_k */
  const void* new_k;    /* optional [B, Hkv, D] */
  const void* new_v;    /* optional [B, Hkv, D] */
  void* out;            /* [B, Hkv, R, D] */
  void* workspace;      /* split-K scratch, >= g4_decode_workspace_size(args) bytes */
  size_t workspace_bytes;
  const G4DecodePrep* prep; /* optional (NULL: q / new_k / new_v are prepared); needs the two-launch path */
  int32_t num_splits;   /* 0 = choose automatically; 1 or 2 = workgroups per (b, kv head), one
                           pass, each owning a slice of the head dim (2: head dim 256; not
                           at head dim 512, which always takes one of the two modes below);
                           G4_DECODE_SPLIT_KEYS = split the key range (bf16, head dims 128/256/512);
                           G4_DECODE_TWO_PASS = scores and values in two launches (rows <= 1024) */
} G4DecodeArgs;

/* num_splits value: split-K over 512-slot key ranges in three launches (scores, values,
 * combine), for long rows over few (b, kv head) pairs. Uses the workspace. The automatic
 * choice takes it for bf16 rows longer than 512 slots when B * Hkv < 256 or when a one-pass
 * row does not fit in LDS, and at head dim 512 for every row beyond the two-launch path's. */
#define G4_DECODE_SPLIT_KEYS (-1)

/* num_splits value: two stream-ordered launches for rows of at most 1024 slots (bf16, head dims
 * 128/256/512): the first scores K chunk by chunk into the workspace, the second forms the exact
 * probabilities and runs the value product, one wave per 16-row block of V^T. Uses the
 * workspace (bf16 scores [B * Hkv][R][512 or 1024]). The automatic choice takes it for such rows
 * when B * Hkv >= 256, and at head dim 512 always. */
#define G4_DECODE_TWO_PASS (-2)

/* Bytes of workspace the call described by args needs (0 when the chosen path uses none). The
 * workspace is plain scratch: no state is kept in it between calls. */
size_t g4_decode_workspace_size(const G4DecodeArgs* args);
int g4_decode_attention(const G4DecodeArgs* args, void* stream);

/*
 * g4_decode_attention without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference: XLA allocates the scratch of its fused computations itself.
 * Same arguments, semantics and results as g4_decode_attention, except that `workspace` must be NULL
 * and `workspace_bytes` 0: the two-launch and split-K paths use a scratch array the library holds,
 * one copy of 32 MiB per device until the process ends (its address is resolved per device by
 * g4_init). A call needing more (g4_decode_workspace_size > 32 MiB, e.g. split-K over more than
 * ~64 (b, kv head) pairs of 32768 slots) is rejected with G4_ERR_WORKSPACE before any launch. Allocates
 * nothing. Every call on a device shares that device's scratch and the scratch keeps no state between
 * calls, so calls that overlap on one GPU (on different streams, or on one stream from different
 * threads without ordering) race; calls ordered on one stream do not.
 */
int g4_decode_attention_noalloc(const G4DecodeArgs* args, void* stream);

/*
 * Causal (optionally sliding-window) prefill attention on the chunk's own K/V. Replaces
 * make_qk_masks (model.py:320-335) + the attention einsums of forward_attention
 * (model.py:496-499) in prefill mode (model.py:455-457, 621-623). Query s of row b attends key
 * t iff t <= s, key_mask[b, t] and (window == 0 or t > s - window) — physical indices, pads
 * count toward the window. Rounding as for g4_decode_attention; a row with no valid key
 * averages all S keys. bf16 runs on MFMA (v_mfma_f32_16x16x32_bf16).
 */
typedef struct G4PrefillArgs {
  int32_t dtype;
  int32_t batch;
  int32_t seq;          /* S (queries = keys) */
  int32_t kv_heads;
  int32_t group;        /* R (bf16: a divisor of 16) */
  int32_t head_dim;     /* bf16: 32, 64, 128, 256 or 512; f32: 8 .. 512 */
  int32_t window;       /* 0 = global (causal only) */
  const uint8_t* key_mask;   /* [B, key_mask_stride] */
  int32_t key_mask_stride;
  const void* q;        /* [B, S, Hkv, R, D] */
  const void* k;        /* key layout with slot_stride = k_stride */
  const void* vt;       /* [B, Hkv, k_stride/8, D, 8] (grouped like cache_vt) */
  int32_t k_stride;     /* >= S, multiple of 64 */
  void* out;            /* [B, S, Hkv, R, D] */
} G4PrefillArgs;

int g4_prefill_attention(const G4PrefillArgs* args, void* stream);

/*
 * Host-side: KV-sharing map (model.py:153-168). layer_types[i] is 0 (sliding) or 1 (full);
 * out[i] = index of the layer whose K/V layer i uses (itself when not shared).
 */
int g4_kv_source_layers(int32_t num_layers, int32_t num_kv_shared_layers, const int32_t* layer_types,
                        int32_t* out);

/* Host-side ring-slot arithmetic (model.py:355-357), the same code the kernels run:
 * out[r] = position held by slot r of a Wc-slot ring after position `last_written` was written
 * (negative = never written). */
int g4_ring_slot_positions(int32_t last_written, int32_t window_capacity, int32_t* out);

/*
 * Next-token sampling fused with the LM head's soft-capping: one step of generate's loop body
 * (sampler.py:265-270) = the key split + _sample_token (sampler.py:145-183), with the capping of
 * forward_lm_head (model.py:676-680) applied on the fly. Per row b:
 *   x       = cast(tanh(l / softcap) * softcap)   (softcap 0: x = l)
 *   (next_key, sample_key) = jax.random.split(key)            threefry2x32, partitionable layout
 *   token   = argmax(x)                                        temperature <= 0
 *           = argmax(x / temperature + gumbel(sample_key)[b])   no proposal (top_k 0, top_p 1)
 *           = proposal_index[b, argmax(proposal[b] + gumbel(sample_key)[b])]   with a proposal
 *   logp    = (x[token] - max(x)) - log(sum(exp(x - max(x))))   (unmodified full-vocab policy)
 * gumbel = -log(-log(u)), u = jax.random.uniform(sample_key, [batch, K], minval=tiny): the bits of
 * element (b, j) are the xor of threefry2x32(sample_key, (hi, lo) of b * K + j). Ties go to the
 * lowest column. `key` is device memory holding 2 uint32 words (jax.random.key_data). With
 * split_key = 1 it is generate's loop state: the draw uses split(key)[1] and a second launch on
 * the stream replaces key by split(key)[0], so graph replays advance it like the reference's
 * while_loop. With split_key = 0 it is _sample_token's key argument: used as is, left unchanged.
 */
typedef struct G4SampleArgs {
  int32_t dtype;                  /* of logits */
  int32_t batch;
  int32_t vocab;
  int32_t proposal_width;         /* K columns of proposal / proposal_index (0 without a proposal) */
  const void* logits;             /* [batch, row_stride] */
  int64_t row_stride;             /* elements, >= vocab */
  float softcap;                  /* 0 = none */
  float temperature;              /* <= 0 = greedy */
  int32_t split_key;              /* 1: split key in place (loop state); 0: key is the sample key */
  uint32_t* key;                  /* device [2]; may be NULL only when greedy */
  const float* proposal;          /* device [batch, K] f32 scores (/ temperature, -inf = cut), or NULL */
  const int32_t* proposal_index;  /* device [batch, K] vocab ids of the proposal columns, or NULL */
  int32_t* token_out;             /* device [batch] */
  float* logp_out;                /* device [batch] */
} G4SampleArgs;

int g4_sample_tokens(const G4SampleArgs* args, void* stream);

/*
 * g4_sample_top_k: the truncated branch of _sample_token (sampler.py:162-183) for 0 < top_k < vocab,
 * top_k <= 256, temperature > 0: the scores s = soft-capped logit / temperature, the top_k largest in
 * descending order (ties: the lower vocab id first, as lax.top_k), the top-p nucleus over them
 * (top_p < 1; the first column always kept), then jax.random.categorical over the top_k columns
 * (Gumbel noise of column j at flat index row * top_k + j) and the drawn column's vocab id; logp is
 * the full unmodified policy's (full-vocab f32 log-softmax of the capped logits). Replaces the
 * torch.sort proposal the host would otherwise build per step. The key as in G4SampleArgs
 * (split_key: split in place after the draw, a second launch). One workgroup per row; no workspace.
 */
typedef struct G4SampleTopKArgs {
  int32_t dtype;        /* of logits: G4_DTYPE_BF16 or G4_DTYPE_F32 */
  int32_t batch;
  int32_t vocab;
  int32_t top_k;        /* 1 .. 256, < vocab */
  const void* logits;   /* [batch, row_stride] */
  int64_t row_stride;   /* elements, >= vocab */
  float softcap;        /* 0 = none (logits already capped) */
  float temperature;    /* > 0 */
  float top_p;          /* (0, 1]; 1 = no nucleus cut */
  int32_t split_key;    /* as G4SampleArgs.split_key */
  uint32_t* key;        /* device [2] */
  int32_t* token_out;   /* device [batch] */
  float* logp_out;      /* device [batch] */
} G4SampleTopKArgs;

int g4_sample_top_k(const G4SampleTopKArgs* args, void* stream);

/*
 * g4_softcap_bf16: out[i] = cast_bf16(tanh(x[i] / cap) * cap) over n bf16 values, the division,
 * tanh and multiply in f32 -- the soft-cap of forward_lm_head (model.py:676-680) as the samplers
 * apply it. cap finite and > 0; x and out 16-byte aligned (out may alias x).
 */
int g4_softcap_bf16(int64_t n, const void* x, float cap, void* out, void* stream);

/*
 * The decode step's LM head with the sampler in its epilogue: l = cast_bf16(x . embed^T) (bf16
 * operands, f32 accumulation; forward_lm_head with the tied embedding, model.py:676-680), then,
 * with token_out given, g4_sample_tokens' draw on l (no proposal) without l leaving the chip:
 * soft-cap, full-vocab log-softmax, the key split (split_key as there) and the greedy /
 * categorical draw of _sample_token (sampler.py:145-183, 265-270). With token_out NULL it is the
 * plain LM head and writes l (before the soft-cap) to logits_out; with both it writes l and draws.
 * Limits: batch 1..256, vocab a multiple of 128, hidden a multiple of 32, vocab * hidden * 2 < 4 GiB;
 * x [batch, hidden] and embed [vocab, hidden] row-major bf16, 16-byte aligned. Sampling needs
 * g4_lm_head_sample_workspace_size() bytes of device workspace (4-byte aligned; one launch at a
 * time per buffer). Two launches on `stream` (the GEMM + epilogue, then the per-row merge).
 */
typedef struct G4LmHeadSampleArgs {
  int32_t batch;
  int32_t vocab;
  int32_t hidden;
  const void* x;          /* [batch, hidden] bf16 */
  const void* embed;      /* [vocab, hidden] bf16 */
  float softcap;          /* 0 = none */
  float temperature;      /* <= 0 = greedy */
  int32_t split_key;      /* as G4SampleArgs.split_key */
  uint32_t* key;          /* device [2]; may be NULL only when greedy */
  int32_t* token_out;     /* device [batch], or NULL: logits only */
  float* logp_out;        /* device [batch] (with token_out) */
  void* logits_out;       /* device [batch, vocab] bf16 before the soft-cap, or NULL (8-byte aligned) */
  void* workspace;        /* device, g4_lm_head_sample_workspace_size() bytes when sampling */
  size_t workspace_bytes;
} G4LmHeadSampleArgs;

size_t g4_lm_head_sample_workspace_size(const G4LmHeadSampleArgs* args);
int g4_lm_head_sample(const G4LmHeadSampleArgs* args, void* stream);

/*
 * Fused elementwise glue of the decoder layer (row-major [rows, cols] arrays, cols <= 4096 for
 * the norms; one pass each, the reference's rounding points kept). dtype = G4_DTYPE_*.
 *
 * g4_rms_norm: out = cast(x * (mean(x^2) + eps)^-0.5 * weight) in f32, weight NULL = no scale.
 *   Replaces forward_rms_norm (model.py:278-285).
 * g4_residual_norm: residual_out = cast(cast(residual + cast(rms(branch) * branch_weight)) *
 *   scalar) (scalar: one f32 value on the device, NULL = none), then, if next_out is given, next_out =
 *   cast(rms(residual_out) * next_weight). residual_out may alias residual. Replaces the
 *   post-norm + residual + layer-scalar steps of forward_decoder_layer (model.py:505-554)
 *   followed by the next pre-norm.
 * g4_gelu_mul: out[r, c] = cast(gelu_tanh(g) * u) in f32 with gate_up[r] = [g (cols) | u (cols)].
 *   Replaces the activation of forward_mlp (model.py:393-396).
 */
int g4_rms_norm(int dtype, int rows, int cols, const void* x, const void* weight, float eps, void* out,
                void* stream);
int g4_residual_norm(int dtype, int rows, int cols, const void* branch, const void* branch_weight,
                     const void* residual, const float* scalar, const void* next_weight, float eps,
                     void* residual_out, void* next_out, void* stream);
int g4_gelu_mul(int dtype, int rows, int cols, const void* gate_up, void* out, void* stream);

/*
 * g4_residual_norm_splitk: g4_residual_norm (bf16) whose branch arrives as ksplit <= 8 f32 partial
 * rows [ksplit][rows][cols] (16-byte aligned): branch = bf16(partials[0] + ... + partials[ksplit-1])
 * added in that order -- the y g4_linear_bf16 would have written. The MLP's down projection at
 * decode (model.py:393-396, 546-553) feeds it without a separate pass over the partials.
 */
int g4_residual_norm_splitk(int rows, int cols, const float* partials, int ksplit, const void* branch_weight,
                            const void* residual, const float* scalar, const void* next_weight, float eps,
                            void* residual_out, void* next_out, void* stream);

/*
 * One decode step's input glue in one launch. Replaces the embedding lookup and scale
 * (model.py:599-600), the key-mask update at the write slot (model.py:608-610) and the rotary
 * tables of forward_gemma4_text (model.py:288-306, 624-627) for S = 1:
 *   x_out[b]       = bf16(f32(embed[tokens[b]]) * embed_scale)      (ids clamped to the table)
 *   key_mask[b, slot[b]] = active[b]                                 (slots outside the row: no write)
 *   cos_out[i][b, d] = cos(f32(positions[b]) * inv_freq[i][d mod rot_dim[i]/2]), sin_out likewise
 * for n_tables <= 2 tables (one per layer type). embed [vocab, hidden] bf16, x_out [batch, hidden]
 * bf16, both 16-byte aligned; hidden a multiple of 8; cos/sin [batch, rot_dim[i]] f32.
 */
typedef struct G4PrologueArgs {
  int32_t batch;
  int32_t hidden;
  int32_t vocab;
  int32_t key_mask_stride;
  const int32_t* tokens;     /* device [B] */
  const int32_t* positions;  /* device [B] logical RoPE positions */
  const uint8_t* active;     /* device [B] (bool) */
  const int32_t* slot;       /* device [B] physical write positions */
  uint8_t* key_mask;         /* device [B, key_mask_stride] */
  const void* embed;
  float embed_scale;
  int32_t n_tables;
  int32_t rot_dim[2];
  const float* inv_freq[2];
  float* cos_out[2];
  float* sin_out[2];
  void* x_out;
} G4PrologueArgs;

int g4_decode_prologue(const G4PrologueArgs* args, void* stream);

/*
 * Decode-step projection: y[m, n] = bf16(sum_k x[m, k] * w[n, k]), f32 accumulation, for the
 * rollout's decode batch (m <= 256 rows). Replaces the q/k/v, o, gate/up and down projections of
 * forward_attention / forward_mlp (model.py:463-482, 500, 393-396) at S = 1, where the reference's
 * einsums (XLA dots, f32 accumulation, bf16 result) multiply one token per row. x [m, k] row-major
 * (16-byte aligned), w [n, k] row-major (the packed, output-major weight), y [m, ldy] (8-byte
 * aligned). n a multiple of 64, k a multiple of 64 * ksplit. ksplit > 1 splits k over that many
 * workgroups per column block; their f32 partial sums are added in split order (workspace
 * [ksplit][m][n] f32, g4_linear_workspace_size bytes). With ksplit > 1 and y == NULL the partial
 * sums are left in the workspace (for g4_residual_norm_splitk).
 * epilogue G4_LINEAR_GELU_MUL (ksplit 1): w holds n = 2F rows, gate rows [0, F) then up rows
 * [F, 2F) (the packed gate/up weight); y [m, F] = bf16(gelu_tanh(g) * u) with g, u the bf16-rounded
 * gate / up products -- forward_mlp's projection and activation (model.py:393-396) in one launch.
 */
#define G4_LINEAR_PLAIN 0
#define G4_LINEAR_GELU_MUL 1

typedef struct G4LinearArgs {
  const void* x;
  const void* w;
  void* y;
  int32_t m;
  int32_t n;
  int32_t k;
  int32_t ldy;
  int32_t ksplit;
  void* workspace;
  size_t workspace_bytes;
  int32_t epilogue;  /* G4_LINEAR_PLAIN or G4_LINEAR_GELU_MUL */
} G4LinearArgs;

size_t g4_linear_workspace_size(const G4LinearArgs* args);
int g4_linear_bf16(const G4LinearArgs* args, void* stream);

/*
 * One iteration of generate's loop body after the draw (sampler.py:279-296), for the batch rows of
 * a rollout at step `step` (0 <= step < max_new):
 *   token = active ? sampled : pad_id;  logp = active ? logp_in : 0
 *   completion_ids[:, step] = token; completion_mask[:, step] = active; rollout_logps[:, step] = logp
 *   active <- active && token is none of eos_ids
 * and the inputs of the decode step that follows it (sampler.py:287-296): next_token = token,
 * next_pos = prompt_lengths + step, next_mask = active before the update (the step's mask).
 * *any_active is set to 1 when a row stays active, else 0 (while_loop's condition, sampler.py:267-
 * 268). completion_ids are int32 (id_bytes 4) or int64 (id_bytes 8), the prompt ids' dtype; masks
 * are one byte per row (0 / 1). batch >= 1. The next_* and any_active pointers may be NULL. One
 * launch of one workgroup on `stream`; it allocates nothing.
 */
typedef struct G4RolloutStepArgs {
  int32_t batch;
  int32_t max_new;
  int32_t step;
  int32_t pad_id;
  int32_t n_eos;
  int32_t id_bytes;               /* 4 or 8 */
  const int32_t* eos_ids;         /* device [n_eos] (NULL when n_eos = 0) */
  const int32_t* sampled;         /* device [batch] */
  const float* logp;              /* device [batch] */
  uint8_t* active;                /* device [batch], updated in place */
  const int32_t* prompt_lengths;  /* device [batch] (needed with next_pos) */
  void* completion_ids;           /* device [batch, max_new] */
  uint8_t* completion_mask;       /* device [batch, max_new] */
  float* rollout_logps;           /* device [batch, max_new] */
  int32_t* next_token;            /* device [batch] or NULL */
  int32_t* next_pos;              /* device [batch] or NULL */
  uint8_t* next_mask;             /* device [batch] or NULL */
  uint8_t* any_active;            /* device [1] or NULL */
} G4RolloutStepArgs;

int g4_rollout_step(const G4RolloutStepArgs* args, void* stream);

/*
 * Rollout weight handoff. g4_convert_f32_to_bf16: out[i] = bf16 bits of in[i], round to nearest
 * even on the raw bits, (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16 — the conversion of
 * inference_device.py:10-45 (device_converter), equal to the astype(bfloat16) of
 * reshard_for_rollout (sharding.py:200-228) on finite values; signed zeros and subnormals are
 * kept. *nonfinite (device int32, may be NULL) is set to 1 when an input is inf / NaN or a result
 * overflows to the inf exponent, and is never cleared: zero it before the call.
 * in and out 16-byte aligned. g4_convert_bf16_to_f32: the exact widening (bits << 16) of
 * reshard_after_rollout's cast back (sharding.py:231-241).
 */
int g4_convert_f32_to_bf16(const float* in, void* out, int64_t n, int32_t* nonfinite, void* stream);
int g4_convert_bf16_to_f32(const void* in, float* out, int64_t n, void* stream);

const char* g4_last_error(void);
const char* g4_version(void);

#ifdef __cplusplus
}
#endif
#endif /* G4_ROLLOUT_H */
