/*
 * sllm_gfx950_decode.h -- a BitNet-b1.58 decode step on one gfx950 GPU.
 *
 * The device-resident form of the reference's forward pass at n = 1
 * (include/saphira_llm/forward.h:23-165, src/forward.c:589-883): the model's
 * tensors uploaded once, the KV cache and every activation kept in HBM, one
 * token per sllm_gfx950_forward. The arithmetic follows the reference
 * operation for operation, so the logits are the reference's bit for bit and
 * so is every int8 activation and int32 dot on the way. Statuses are those of
 * sllm_gfx950.h (the reference's sllm_status values where one applies).
 *
 * The library must be open (sllm_gfx950_open). Work is enqueued on the
 * library stream; calls that return host data synchronise it.
 */
#ifndef SAPHIRA_AMD_SLLM_GFX950_DECODE_H
#define SAPHIRA_AMD_SLLM_GFX950_DECODE_H

#include <saphira_amd/sllm_gfx950.h>

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One block's tensors in host memory, as the reference's sllm_layer holds
 * them after sllm_model_load (src/forward.c:397-430): I2_S matrices with
 * their 32-byte tails, f32 norm weights. */
typedef struct sllm_gfx950_layer_desc {
    const uint8_t *wq, *wk, *wv, *wo, *w_gate, *w_up, *w_down;
    const float   *attn_norm, *attn_sub_norm, *ffn_norm, *ffn_sub_norm;
} sllm_gfx950_layer_desc;

/* The model's hyper-parameters and tensors (the fields of sllm_model the
 * forward pass reads, src/forward.c:318-455). tok_embd is n_vocab rows of
 * n_embd binary16 values, the token embedding and the tied output
 * projection. */
typedef struct sllm_gfx950_model_desc {
    int32_t  n_layer, n_embd, n_ff, n_head, n_head_kv, n_rot, n_vocab;
    float    eps;          /* RMSNorm epsilon */
    float    rope_base;    /* RoPE frequency base */
    const uint16_t *tok_embd;
    const float    *output_norm;
    const sllm_gfx950_layer_desc *layers;   /* n_layer entries */
} sllm_gfx950_model_desc;

typedef struct sllm_gfx950_model sllm_gfx950_model;
typedef struct sllm_gfx950_ctx   sllm_gfx950_ctx;

/* Largest shapes the decode kernels take: head dimension, query heads per KV
 * head, n_embd / n_ff (the slab GEMV's LDS row), and query heads per KV head
 * times n_ctx (the softmax rows held in LDS). */
#define SLLM_GFX950_DEC_MAX_HEAD_DIM 128
#define SLLM_GFX950_DEC_MAX_GQA      4
#define SLLM_GFX950_DEC_MAX_WIDTH    7168
#define SLLM_GFX950_DEC_MAX_GQA_CTX  16384
/* Most tokens in one sllm_gfx950_forward_chunk (the reference's
 * SLLM_MAX_CHUNK, include/saphira_llm/forward.h:90, is 256). */
#define SLLM_GFX950_DEC_MAX_CHUNK    512
/* Tokens a greedy generation keeps enqueued ahead of the host
 * (sllm_gfx950_ctx_set_inflight). */
#define SLLM_GFX950_DEC_MAX_INFLIGHT     64
#define SLLM_GFX950_DEC_DEFAULT_INFLIGHT 8

/*
 * sllm_model_load (forward.h:33) for the device: copies every tensor of
 * `desc` into device memory, byte for byte. The host buffers may be freed
 * afterwards. Shapes are checked as src/forward.c:306-455 checks them
 * (I2_S widths multiples of 128) plus the kernel limits above:
 * SLLM_GFX950_ERR_TENSOR_SHAPE or SLLM_GFX950_ERR_TOO_LARGE.
 */
int  sllm_gfx950_model_upload(const sllm_gfx950_model_desc *desc, sllm_gfx950_model **out);
void sllm_gfx950_model_free(sllm_gfx950_model *m);

/*
 * sllm_gguf_open_memory (include/saphira_llm/gguf.h:144) followed by
 * sllm_model_load (forward.h:32), then sllm_gfx950_model_upload: a GGUF v3
 * image of a bitnet-b1.58 model in host memory onto the device. The image is
 * read in place and may be freed afterwards. A file is accepted or refused
 * as the reference accepts or refuses it, with its status: the container
 * (SLLM_GFX950_ERR_GGUF_*, SLLM_GFX950_ERR_TOO_LARGE past the reference's
 * count and length limits), then the model (SLLM_GFX950_ERR_ARCH,
 * SLLM_GFX950_ERR_KV_MISSING for an absent or mistyped hyper-parameter,
 * SLLM_GFX950_ERR_TENSOR_SHAPE for an absent or misshapen tensor); then the
 * kernel limits of sllm_gfx950_model_upload.
 */
int  sllm_gfx950_model_load_gguf(const void *image, size_t size, sllm_gfx950_model **out);
/* The same from a file, mapped read-only (sllm_gguf_open, gguf.h:141);
 * SLLM_GFX950_ERR_IO if it cannot be opened or mapped, TRUNCATED if empty. */
int  sllm_gfx950_model_load_gguf_file(const char *path, sllm_gfx950_model **out);
/*
 * The host half of sllm_gfx950_model_load_gguf, needing no device: parse and
 * check the image and fill `desc` with pointers into it; layers must hold 64
 * entries (the reference's SLLM_LAYER_MAX, src/forward.c:45).
 */
int  sllm_gfx950_gguf_describe(const void *image, size_t size, sllm_gfx950_model_desc *desc,
                               sllm_gfx950_layer_desc *layers);

/*
 * sllm_ctx_new (forward.h:46): a KV cache of n_ctx positions
 * ([layer][head_kv][pos][head_dim] f32, as src/forward.c:466-518) and the
 * activations, all on the device, plus the RoPE table for positions
 * 0..n_ctx-1 (cos / sin built with the host C library, as the reference's
 * src/ops.c:467-549 builds them per token).
 */
int  sllm_gfx950_ctx_new(const sllm_gfx950_model *m, int32_t n_ctx, sllm_gfx950_ctx **out);
void sllm_gfx950_ctx_free(sllm_gfx950_ctx *c);
/* sllm_ctx_reset (forward.h:50): zero the live cache prefix, n_past = 0 */
int  sllm_gfx950_ctx_reset(sllm_gfx950_ctx *c);
int32_t sllm_gfx950_ctx_n_past(const sllm_gfx950_ctx *c);

/*
 * sllm_forward (forward.h:83): one token at `pos`. Refused as the reference
 * refuses it (src/forward.c:592-608): pos < n_past (rewinding) or
 * pos >= n_ctx, token outside [0, n_vocab) -> SLLM_GFX950_ERR_ARG. logits:
 * n_vocab floats of host memory, or NULL to leave them on the device (read
 * them with sllm_gfx950_ctx_logits). Returns after the step has been
 * enqueued, or -- logits given -- completed.
 */
int  sllm_gfx950_forward(const sllm_gfx950_model *m, sllm_gfx950_ctx *c, int32_t token, int32_t pos,
                         float *logits);

/*
 * sllm_forward_chunk (forward.h:93-109): n tokens as one chunk at positions
 * base .. base + n - 1, every projection one int8-MFMA GEMM over the n
 * quantised rows, with the logits of the token-by-token path bit for bit
 * (src/forward.c:589-835; tests/test_phase5.c:85-150). Refused as the
 * reference refuses it: n < 1 or n > SLLM_GFX950_DEC_MAX_CHUNK, base <
 * n_past, base + n > n_ctx, a token out of range -> SLLM_GFX950_ERR_ARG.
 * logits: n * n_vocab floats of host memory (row t for token t), or NULL
 * to compute the last token's logits only and leave them on the device. The
 * last token's logits and argmax are kept as after sllm_gfx950_forward. n = 1
 * runs the decode step.
 */
int  sllm_gfx950_forward_chunk(const sllm_gfx950_model *m, sllm_gfx950_ctx *c, const int32_t *tokens,
                               int32_t n, int32_t base, float *logits);

/*
 * sllm_forward_prefill_chunked (forward.h:111-113, src/forward.c:846-868):
 * tokens 0 .. n - 1 at positions 0 .. n - 1 in chunks of `chunk`; logits:
 * n * n_vocab floats or NULL. chunk < 1 or above the limit ->
 * SLLM_GFX950_ERR_ARG; n > n_ctx -> SLLM_GFX950_ERR_TOO_LARGE.
 */
int  sllm_gfx950_forward_prefill_chunked(const sllm_gfx950_model *m, sllm_gfx950_ctx *c, const int32_t *tokens,
                                         int32_t n, int32_t chunk, float *logits);

/*
 * sllm_generate_greedy (forward.h:124): forward the prompt, then n_new
 * tokens, each the argmax (src/forward.c:876-883) of the previous logits;
 * out receives the n_new ids. The token loop runs on the device: each step's
 * output kernel feeds the next token itself, so the host enqueues the whole
 * generation and synchronises once. SLLM_GFX950_ERR_TOO_LARGE past n_ctx.
 */
int  sllm_gfx950_generate_greedy(const sllm_gfx950_model *m, sllm_gfx950_ctx *c, const int32_t *prompt,
                                 int32_t n_prompt, int32_t n_new, int32_t *out);

/* The device copy of the last logits (n_vocab floats), and their argmax
 * (synchronises). */
const float *sllm_gfx950_ctx_logits(const sllm_gfx950_ctx *c);
int  sllm_gfx950_ctx_argmax(sllm_gfx950_ctx *c, int32_t *token);

/*
 * sllm_state_load (forward.h:162, src/forward.c:1040-1121) without the file:
 * fill positions [0, n_pos) of the cache from host memory -- k and v laid
 * out [layer][head_kv][pos][head_dim] with n_pos positions per head --, clear
 * positions [n_pos, n_ctx) of every (layer, KV head), restore the last
 * position's logits (n_vocab floats, the state file's tail) and set n_past =
 * n_pos. An empty-prompt sllm_gfx950_generate_greedy then continues from the
 * restored logits' argmax, as the reference's does (src/forward.c:909-912).
 * logits may be NULL: the context then has no last logits, and an
 * empty-prompt generate is refused (SLLM_GFX950_ERR_ARG) until a forward.
 */
int  sllm_gfx950_ctx_kv_load(sllm_gfx950_ctx *c, const float *k, const float *v, int32_t n_pos,
                             const float *logits);

/*
 * How many tokens sllm_gfx950_generate_greedy keeps enqueued ahead of the
 * host (1 .. SLLM_GFX950_DEC_MAX_INFLIGHT, default
 * SLLM_GFX950_DEC_DEFAULT_INFLIGHT): before enqueueing token i it waits for
 * token i - tokens to finish. Two or more keep the device busy; the bound
 * keeps the number of dispatches outstanding at any time to tokens times a
 * token's launches, where an unbounded loop would queue the whole
 * generation at once.
 */
int  sllm_gfx950_ctx_set_inflight(sllm_gfx950_ctx *c, int32_t tokens);

/*
 * Capture one token's launches in a HIP graph and replay it for every later
 * token (on = 1), or launch them one by one (on = 0, the default). The
 * results are the same; the graph saves host launch time.
 */
int  sllm_gfx950_ctx_set_graph(sllm_gfx950_ctx *c, int on);

/*
 * Parity tracing. dots: device memory for every projection's raw int32 dots
 * of one token, per layer q, k, v, o, gate, up, down (n_layer * (2*n_embd +
 * 2*gqa + 3*n_ff) + ... = sllm_gfx950_trace_dots(m) values); acts: device
 * memory for 4 * n_layer activations (per layer: attn, o, ffn, down
 * quantisation). NULL, NULL stops tracing. Each forward overwrites them.
 */
size_t sllm_gfx950_trace_dots(const sllm_gfx950_model *m);
int  sllm_gfx950_ctx_trace(sllm_gfx950_ctx *c, int32_t *dots, sllm_gfx950_act *acts);

#ifdef __cplusplus
}
#endif

#endif /* SAPHIRA_AMD_SLLM_GFX950_DECODE_H */
