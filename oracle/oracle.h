/*
 * CPU oracle for the Gemma-3-1B Q4_0 forward path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker: it is loaded
 * by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg,
 * and by nothing else. The product library never links, loads or calls it.
 *
 * It restates the reference's WGSL arithmetic on the CPU, rounding point for
 * rounding point (each function cites the reference file:line it follows):
 * every explicit WGSL fma is std::fma, every other multiply and add rounds
 * separately (built with -ffp-contract=off), and every reduction keeps the
 * reference's tree or chain order.
 *
 * The reference leaves a few rounding points to WGSL built-ins whose results
 * are implementation-defined (inverseSqrt, cos, sin, exp2, exp, dot). This
 * oracle fixes each one to a stated definition; the HIP kernels implement the
 * same definitions, so the two agree bit for bit:
 *   dot(a, b)       ((a0*b0 + a1*b1) + a2*b2) + a3*b3, each op rounded
 *   inverseSqrt(x)  1 / sqrt(x), both correctly rounded f32 operations
 *   exp2(x)         orc_exp2 (Cody-Waite split, degree-7 polynomial)
 *   cos, sin        orc_cos / orc_sin (quadrant split, Taylor to r^12 / r^11)
 *   exp(x), x <= 0  the reference's own explicit exp_nonpositive
 * The accuracy of each definition against libm in f64 is pinned by the CPU
 * tests; the exact bits of the reference's built-ins on its own GPUs are not
 * defined and stay "parity unpinned".
 *
 * How each function is pinned (tests/test_oracle.py):
 *   orc_q4_0_unpack   the reference's fixture valid.gguf; every code x every
 *                     finite f16 scale against the exact product
 *   orc_f16_*         all 65,536 halves; saturate + round-to-nearest-even
 *                     against numpy's IEEE conversion, ties included
 *   orc_gemv/gated    exact integer results; range boundaries and their order
 *                     (2^24 + 1 + 1 constructions); fma chaining; the
 *                     gamma(2K) bound against f64
 *   orc_norm_row      f64 within 2^-18 (the reference's design margin)
 *   orc_rope_turns    the f64 closed form, bit for bit
 *   orc_rope_row      f64 rotation; the cache as numpy's f16 of the clamp
 *   orc_attention_row f64 softmax attention; keys outside the window inert
 *   orc_gather_row    the dequantized row times the scale
 *   orc_q8_0_unpack,  every code x every finite f16 scale (and minimum)
 *   orc_q4_1_unpack   against the exact value rounded once to f32; the
 *                     fixture-style blocks their generator states
 *   orc_gemv_format   Q4_0 equal to orc_gemv; exact integer results for
 *                     Q8_0 and Q4_1 (the order is orc_gemv's, pinned above)
 *   orc_norm_row_added  hidden after = hidden before + added, bit for bit;
 *                     added against the f64 post-norm within 2^-18
 *   orc_attention_row_scores  the output is orc_attention_row's bit for
 *                     bit; scores against f64 dots, m their maximum, l the
 *                     f64 sum of exp2(s - m); untouched past the keys read
 *   orc_model_residuals, orc_model_capture  the model's own intermediates
 *                     (pinned through the functions above and the model's
 *                     logits); the capture store's layout is pinned by the
 *                     reference's counts in tests/test_capture.py
 *   orc_edit_row      the edit kernel contract (edit_kernel_test.cpp:1-21)
 *   orc_topk          brute-force stable sort in the total order
 *   orc_philox        Random123 known answers; orc_mulhi against 64-bit
 *   orc_draw          greedy and the uniform's closed form; the inverse
 *                     transform against f64
 *   orc_inverse_sqrt  bit for bit against numpy's correctly rounded ops
 *   orc_dot4          order by a 2^24 + 1 + 1 construction
 *   orc_exp2, orc_exp_nonpositive, orc_gelu_tanh, orc_cos, orc_sin
 *                     accuracy against f64 only: their bits, as the
 *                     reference's built-ins give them, are parity unpinned
 *
 * Weights are blocks as GGUF stores them, a matrix of N rows of K being
 * N * K / 32 blocks, row-major: Q4_0 (format 2) 18 bytes, an fp16 scale d
 * then 16 code bytes; Q4_1 (3) 20 bytes, d, an fp16 minimum m, 16 code
 * bytes; Q8_0 (8) 34 bytes, d then 32 signed codes.
 */
#ifndef FRIZZLE_ORACLE_H
#define FRIZZLE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- numerics -------------------------------------------------------- */
float orc_exp_nonpositive(float x);
float orc_gelu_tanh(float g);
float orc_exp2(float x);
float orc_cos(float angle);
float orc_sin(float angle);
float orc_inverse_sqrt(float x);
uint16_t orc_f16_pack(float x);
float orc_f16_unpack(uint16_t h);
float orc_dot4(const float* a, const float* b);

/* ---- formats and products --------------------------------------------- */
void orc_q4_0_unpack(const uint8_t* block, float out[32]);
void orc_q4_1_unpack(const uint8_t* block, float out[32]);
void orc_q8_0_unpack(const uint8_t* block, float out[32]);
/* Bytes of one block of GGUF format `format` (2, 3 or 8); 0 for others. */
int orc_block_bytes(int format);
void orc_gemv_format(int format, const uint8_t* w, int rows, int cols,
                     const float* x, float* y);
void orc_gemv(const uint8_t* w, int rows, int cols, const float* x,
              float* y);
void orc_gated(const uint8_t* gate, const uint8_t* up, int rows, int cols,
               const float* x, float* act);

/* ---- per-row kernels -------------------------------------------------- */
void orc_norm_row(const float* gain, const float* post_gain, int add,
                  int post_norm, float post_scale, float epsilon, int width,
                  float* hidden, const float* output, float* normed);
/* orc_norm_row, also giving the vector the add added (when added is not
 * null and add is set). */
void orc_norm_row_added(const float* gain, const float* post_gain, int add,
                        int post_norm, float post_scale, float epsilon, int width,
                        float* hidden, const float* output, float* normed, float* added);
void orc_rope_turns(float base, int head_dim, float* turns);
void orc_rope_row(int position, int slots, int head_dim, int query_heads,
                  int kv_heads, float epsilon, const float* turns,
                  const float* query_gain, const float* key_gain,
                  float* query, const float* key, const float* value,
                  uint16_t* key_cache, uint16_t* value_cache);
void orc_attention_row(int position, int window, int slots, int head_dim,
                       int query_heads, int kv_heads, float scale_log2e,
                       const float* query, const uint16_t* key_cache,
                       const uint16_t* value_cache, float* out);
/* orc_attention_row, also giving each head's scores of the keys its query
 * reads (key earliest + i at scores[h * keys + i], earliest =
 * p + 1 - min(p + 1, keys)) and its final (m, l) at stats[2h], [2h + 1]. */
void orc_attention_row_scores(int position, int window, int slots, int head_dim,
                              int query_heads, int kv_heads, float scale_log2e,
                              const float* query, const uint16_t* key_cache,
                              const uint16_t* value_cache, float* out, float* scores,
                              int keys, float* stats);
void orc_gather_row(const uint8_t* table, int width, uint32_t token,
                    float scale, float* hidden);
void orc_gather_row_format(int format, const uint8_t* table, int width,
                           uint32_t token, float scale, float* hidden);
void orc_edit_row(const uint32_t* table, int layer, uint32_t position,
                  int width, float* activation);
void orc_topk(const float* logits, int count, uint32_t* bits,
              uint32_t* ids);
void orc_philox(const uint32_t counter[4], const uint32_t key[2],
                uint32_t out[4]);
uint32_t orc_mulhi(uint32_t a, uint32_t b);
void orc_draw(const uint32_t* cand_bits, const uint32_t* cand_ids,
              uint32_t count, uint32_t top_k, float temperature, float top_p,
              float min_p, float log_min_p, uint32_t counter,
              uint32_t seed_lo, uint32_t seed_hi, uint32_t record[4]);

/* ---- the model -------------------------------------------------------- */
/* Shapes of a Gemma-3 model. Layer l is global (full context, global rope
 * base) when l % pattern == pattern - 1, else it slides over `window`. */
typedef struct orc_config {
  int hidden;      /* 1152 */
  int ffn;         /* 6912 */
  int head_dim;    /* 256 */
  int query_heads; /* 4 */
  int kv_heads;    /* 1 */
  int layers;      /* 26 */
  int vocab;       /* 262144 */
  int window;      /* 512 */
  int pattern;     /* 6 */
  int context;     /* positions a global layer's cache holds */
  int local_slots; /* a window layer's ring: window + 512 + reserve */
  float rope_local;
  float rope_global;
  float epsilon;
  int embedding_format; /* the tied embedding/head's format (0 means Q4_0) */
} orc_config;

/* Borrowed pointers to one layer's weights (GGUF Q4_0 blocks, the down
 * matrix in `down_format` (0 means Q4_0); F32 gains). */
typedef struct orc_layer_weights {
  const uint8_t* q;    /* query_heads*head_dim rows of hidden */
  const uint8_t* k;    /* kv_heads*head_dim rows of hidden */
  const uint8_t* v;
  const uint8_t* o;    /* hidden rows of query_heads*head_dim */
  const uint8_t* gate; /* ffn rows of hidden */
  const uint8_t* up;
  const uint8_t* down; /* hidden rows of ffn */
  const float* attn_norm;
  const float* q_norm;
  const float* k_norm;
  const float* post_attn_norm;
  const float* ffn_norm;
  const float* post_ffn_norm;
  int down_format;
} orc_layer_weights;

typedef struct orc_model orc_model;

orc_model* orc_model_create(const orc_config* config,
                            const orc_layer_weights* layers,
                            const uint8_t* embedding, const float* output_norm);
void orc_model_destroy(orc_model* m);
/* A second model in the same state (caches, edits, last token's values),
 * over the same weights: many continuations of one prompt run it once. */
orc_model* orc_model_clone(const orc_model* m);
/* The edit table (u32 words, the reference's layout) used from now on. */
void orc_model_set_edits(orc_model* m, const uint32_t* table, int words);
/* One token at `position` through every layer; writes the logits
 * (vocab floats) when `logits` is not null. */
void orc_model_token(orc_model* m, uint32_t token, int position,
                     float* logits);
/* A prefill block: n (1 .. 512) tokens from `position`, layer by layer, as
 * one step of the reference's prefill runs them. Each row's arithmetic is
 * orc_model_token's; each layer appends the block's keys and values before
 * any row attends (a sliding layer's ring holds at least window + 512
 * slots, so no row's window is overwritten). Writes the last row's logits
 * when `logits` is not null; the residuals are the last row's. The capture
 * store is not written (orc_model_token writes it). Pinned by equality with
 * orc_model_token, token by token, in tests/test_oracle_pins.py. */
void orc_model_block(orc_model* m, const uint32_t* tokens, int n, int position,
                     float* logits);
/* The last layer's output row after the final norm (hidden floats). */
const float* orc_model_normed(const orc_model* m);
/* [layers][hidden]: for the last token, the residual entering each layer
 * (X after the add of the layer's first norm; layer 0's is the embedding). */
const float* orc_model_residuals(const orc_model* m);
/* The capture store's values for the last token, kept while capture is on
 * (src/core/capture/capture.h:12-34): slot 0 neurons, 1 residual,
 * 2 attention_added, 3 mlp_added, 4 query, 5 weights, 6 stats, 7 readout,
 * as 32-bit words; *words gets the slot's width. */
void orc_model_set_capture(orc_model* m, int on);
const uint32_t* orc_model_capture(const orc_model* m, int layer, int slot, int* words);
/* Read access to layer l's F16 key and value cache, slots x kv x head_dim. */
const uint16_t* orc_model_key_cache(const orc_model* m, int layer);
const uint16_t* orc_model_value_cache(const orc_model* m, int layer);
int orc_model_slots(const orc_model* m, int layer);

#ifdef __cplusplus
}
#endif

#endif
