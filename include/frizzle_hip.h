/*
 * frizzle_hip.h — the C ABI of the MI355X (gfx950) backend for the Gemma-3-1B
 * Q4_0 forward path.
 *
 * It takes the place of the reference's executor boundary: the Dawn/WebGPU
 * device (src/core/gpu/device.h:132-198), buffer residency and upload
 * (src/core/residency/upload.h:263-300), and the program that runs a step's
 * launches (src/core/kernels/program.h:330-402), together with the WGSL
 * kernels those launches name. Everything here is plain C: opaque handles,
 * plain pointers and sizes, an int status (0 = ok) and a thread-local message
 * from frz_last_error(). Nothing throws across this boundary.
 *
 * Device pointers ("dev") are addresses from frz_alloc on the same device.
 * Host pointers are ordinary memory. Unless stated, calls enqueue work on the
 * device's one stream and return without waiting; frz_sync waits.
 */
#ifndef FRIZZLE_HIP_H
#define FRIZZLE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes, as the reference's ProgramError (src/core/kernels/program.h:
 * 264-278) plus argument refusals. */
enum frz_status {
  FRZ_OK = 0,
  FRZ_ERR_ARGUMENT = 1,    /* refused before any work: a bad size or shape */
  FRZ_ERR_DEVICE = 2,      /* no device, or a HIP call failed */
  FRZ_ERR_BUILD = 3,       /* a program could not be built */
  FRZ_ERR_STEP = 4,        /* a step failed on the device */
  FRZ_ERR_DEVICE_LOST = 5, /* the device stopped answering */
  FRZ_ERR_CANCELLED = 6
};

/* The message of the calling thread's last failed call ("" when none). */
const char* frz_last_error(void);

/* ---- device (replaces gpu::Device::request, src/core/gpu/device.h:152-198) */
typedef struct frz_device frz_device;

typedef struct frz_limits {
  char name[64];              /* the device's architecture name, "gfx950" */
  uint64_t memory_bytes;      /* HBM on the device */
  int compute_units;
  int lds_bytes_per_block;
} frz_limits;

int frz_open(int ordinal, frz_device** out, frz_limits* limits);
void frz_close(frz_device* dev);
int frz_sync(frz_device* dev);

/* ---- buffers (replaces residency::Upload::begin/write/buffer,
 *      src/core/residency/upload.h:276-300) --------------------------------- */
int frz_alloc(frz_device* dev, uint64_t bytes, void** dev_ptr);
int frz_free(frz_device* dev, void* dev_ptr);
/* Host to device and back; both wait for the copy. */
int frz_write(frz_device* dev, void* dev_dst, const void* host_src, uint64_t bytes);
int frz_read(frz_device* dev, void* host_dst, const void* dev_src, uint64_t bytes);
int frz_fill_zero(frz_device* dev, void* dev_dst, uint64_t bytes);
/* Device to device; waits for the copy. */
int frz_copy(frz_device* dev, void* dev_dst, const void* dev_src, uint64_t bytes);

/* The Q4_0 upload transform (replaces residency::PieceWriter,
 * src/core/residency/piece_writer.h:44-60, with the device layout of
 * src/core/formats/device_layout.h:114-115): `blocks` GGUF Q4_0 blocks of 18
 * bytes (an fp16 scale, then 16 code bytes) become two streams, every
 * block's 16 code bytes, then every block's scale. Host to host. */
int frz_q4_0_split(const void* gguf_blocks, uint64_t blocks, void* codes_out,
                   void* scales_out);
/* The same transform for any weight format the library computes in (GGUF
 * numbers: FRZ_FORMAT_Q4_0 2, FRZ_FORMAT_Q4_1 3, FRZ_FORMAT_Q8_0 8), with
 * the device layouts of src/core/formats/device_layout.h:114-119: Q4_0 16
 * code bytes and one scale half a block; Q4_1 16 code bytes and two halves
 * (d, m); Q8_0 32 code bytes and one half. GGUF blocks are 18, 20 and 34
 * bytes. */
#define FRZ_FORMAT_F32 0
#define FRZ_FORMAT_Q4_0 2
#define FRZ_FORMAT_Q4_1 3
#define FRZ_FORMAT_Q8_0 8
int frz_block_split(int format, const void* gguf_blocks, uint64_t blocks,
                    void* codes_out, void* scales_out);

/* ---- one kernel at a time (the reference's launchers, each a Launch of
 *      src/core/kernels/interface.h:320-363, run alone as the kernel contract
 *      tests do, tests/support/scratch_program.h:62-80) -----------------------
 * A Q4_0 matrix is `rows` rows of `cols` weights in the split layout above:
 * codes (rows * cols / 32 * 16 bytes) and scales (rows * cols / 32 halves).
 * `tokens` rows of input are processed from `position`. */

/* y[t][o] = sum_k W[o][k] x[t][k] in the reference's order of addition
 * (src/core/kernels/matmul/matmul.wgsl:154-244, 390-465): the decode form
 * when tokens == 1 or last_token, the tiled form otherwise. */
int frz_op_gemv(frz_device* dev, const void* codes, const void* scales,
                int rows, int cols, const float* x, int x_stride, float* y,
                int y_stride, uint32_t tokens, int last_token);
/* The same product over Q4_1 or Q8_0 weights as well (codes and scales in
 * frz_block_split's layout): a format supplies only its unpack
 * (src/core/formats/format.h; q4_1.wgsl, q8_0.wgsl), the order of addition
 * is the same. */
int frz_op_gemv_format(frz_device* dev, int format, const void* codes,
                       const void* scales, int rows, int cols, const float* x,
                       int x_stride, float* y, int y_stride, uint32_t tokens,
                       int last_token);
/* act[t][j] = gelu_tanh(gate_j) * up_j with layer `layer`'s pins applied at
 * position + t (matmul.wgsl:247-276 and src/core/edit/edit.wgsl:55-76 fused);
 * edits_dev may be null for none. */
int frz_op_gated(frz_device* dev, const void* gate_codes,
                 const void* gate_scales, const void* up_codes,
                 const void* up_scales, int rows, int cols, const float* x,
                 float* act, uint32_t tokens, uint32_t position,
                 const uint32_t* edits_dev, int layer);
/* The fast prefill mode's products (FRZ_PREFILL_BF16), op by op: y = W x
 * over bf16 pair operands, K split over `splits` (1 to 16; 0: as the model
 * splits it) and the splits added in order; and the gated product with its
 * pins (rows a multiple of 16). The weights are unpacked into bf16 pair
 * planes and x split into pair planes first. Within about 2^-16 of each
 * product of the exact sum, not the reference's order (no counterpart in
 * the reference, which computes in fp32). */
int frz_op_gemm_bf16(frz_device* dev, int format, const void* codes, const void* scales,
                     int rows, int cols, const float* x, int x_stride, float* y, int y_stride,
                     uint32_t tokens, int splits);
int frz_op_gated_bf16(frz_device* dev, const void* gate_codes, const void* gate_scales,
                      const void* up_codes, const void* up_scales, int rows, int cols,
                      const float* x, float* act, uint32_t tokens, uint32_t position,
                      const uint32_t* edits_dev, int layer);
/* RMSNorm with the residual add and post-norm (kernels/norm/norm.wgsl:96-198).
 * post_gain null: no add; otherwise hidden += postnorm(output). last_token:
 * the step's last row only. */
int frz_op_norm(frz_device* dev, const float* gain, const float* post_gain,
                const float* output, float* hidden, float* normed, int width,
                float epsilon, uint32_t tokens, int last_token);
/* QK-norm, rope and the F16 KV append (kernels/rope/rope.wgsl,
 * rope_cache.wgsl). turns: head_dim/2 floats from frz_rope_turns. Rows of
 * query/key/value are q_stride / kv_stride floats apart. */
int frz_op_rope(frz_device* dev, const float* turns, const float* query_gain,
                const float* key_gain, float* query, const float* key,
                const float* value, int q_stride, int kv_stride,
                uint16_t* key_cache, uint16_t* value_cache, int slots,
                int head_dim, int query_heads, int kv_heads, float epsilon,
                uint32_t position, uint32_t tokens);
/* Attention over the F16 cache (kernels/attention/attention.wgsl:166-438).
 * out: tokens x query_heads x head_dim. */
int frz_op_attention(frz_device* dev, const float* query, int q_stride,
                     const uint16_t* key_cache, const uint16_t* value_cache,
                     float* out, int slots, int window, int head_dim,
                     int query_heads, int kv_heads, float scale,
                     uint32_t position, uint32_t tokens);
/* One decode token's QK-norm, rope and F16 KV append fused with its attention
 * (rope.wgsl + rope_cache.wgsl + attention.wgsl, one launch): qkv holds the
 * token's 4 x 256 query, 256 key and 256 value floats; head_dim 256, 4 query
 * heads on 1 key-value head. */
int frz_op_rope_attention(frz_device* dev, const float* qkv, const float* turns,
                          const float* query_gain, const float* key_gain,
                          uint16_t* key_cache, uint16_t* value_cache, float* out,
                          int slots, int window, float epsilon, float scale,
                          uint32_t position);
/* The same as frz_op_rope_attention, allocating nothing: no counterpart in
 * the reference. For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The chunk states live in a static workspace of 931,840 bytes that each
 * device holds until the process ends, so window and slots may reach at
 * most 224 chunks (14,272 keys; FRZ_ERR_ARGUMENT beyond). Every call on one
 * device shares that workspace, which keeps the last call's contents (each
 * call writes every state it reads): calls that overlap on one device race. */
int frz_op_rope_attention_noalloc(frz_device* dev, const float* qkv, const float* turns,
                                  const float* query_gain, const float* key_gain,
                                  uint16_t* key_cache, uint16_t* value_cache, float* out,
                                  int slots, int window, float epsilon, float scale,
                                  uint32_t position);
/* Embedding rows times scale (kernels/gather/gather.wgsl:25-48). */
int frz_op_gather(frz_device* dev, const void* codes, const void* scales,
                  int rows, int cols, const uint32_t* ids, uint32_t tokens,
                  float scale, float* hidden);
/* The same from a Q4_0 or Q8_0 table (gather.h: the file's embedding is
 * Q8_0). */
int frz_op_gather_format(frz_device* dev, int format, const void* codes,
                         const void* scales, int rows, int cols,
                         const uint32_t* ids, uint32_t tokens, float scale,
                         float* hidden);
/* One layer's pins alone (src/core/edit/edit.wgsl:55-76). */
int frz_op_edit(frz_device* dev, const uint32_t* edits_dev, int layer,
                float* act, int width, uint32_t position, uint32_t tokens);
/* Top-64 (kernels/topk/topk.wgsl): candidates_dev gets 64 x {bits, token}. */
int frz_op_topk(frz_device* dev, const float* logits, int count,
                uint32_t* candidates_dev);

/* Sampling settings of a turn (src/core/policy/policy.h:41-46) with its seed
 * (policy::Seed), as sampler::apply puts them in a step
 * (src/core/sampler/sampler.cpp:51-62). */
typedef struct frz_sampling {
  uint32_t top_k;
  float temperature;
  float top_p;
  float min_p;
  uint64_t seed;
} frz_sampling;

/* The draw (src/core/sampler/draw.wgsl:77-170): record_dev gets
 * {token, failed, u bits, 0} for the position position + tokens. */
int frz_op_draw(frz_device* dev, const uint32_t* candidates_dev,
                const frz_sampling* sampling, uint32_t position,
                uint32_t tokens, uint32_t* record_dev);

/* The shared numerics on the device, for their contract tests: which = 0
 * exp2, 1 cos, 2 sin, 3 inverse sqrt, 4 gelu_tanh, 5 exp_nonpositive,
 * 6 f16 pack (out holds the halves' bits as floats' low 16 bits, via
 * uint32), 7 sqrt, 8 division in[2i] / in[2i+1]. */
int frz_op_numerics(frz_device* dev, int which, const float* in_dev,
                    float* out_dev, int n);

/* Times the decode GEMV over `copies` distinct weight copies in turn (so
 * the weights stream from HBM, not a cache): with `graph`, one launch per
 * copy captured in a HIP graph and replayed until `iters` launches; without,
 * `iters` launches on the stream. Timed with HIP events on the launching
 * stream; writes the mean microseconds a launch. No counterpart in the
 * reference, which times nothing (measurement only). */
int frz_bench_gemv(frz_device* dev, const void* const* codes,
                   const void* const* scales, int copies, int rows, int cols,
                   const float* x, float* y, int iters, int graph,
                   double* us_per_launch);
/* The same for the gated product (gate and up copies in turn). */
int frz_bench_gated(frz_device* dev, const void* const* gate_codes,
                    const void* const* gate_scales,
                    const void* const* up_codes, const void* const* up_scales,
                    int copies, int rows, int cols, const float* x, float* act,
                    int iters, int graph, double* us_per_launch);

/* Floors, measured the same way: an empty kernel launched `iters` times
 * (with `graph`, 64 launches captured and replayed), and a streaming read of
 * `bytes` (a multiple of 16) from each of `copies` device buffers in turn, by
 * 1,024 workgroups, xor-folded into sink[0..1023] (device memory of 1,024
 * words). No counterpart in the reference (measurement only). */
int frz_bench_launch_floor(frz_device* dev, int iters, int graph,
                           double* us_per_launch);
int frz_bench_stream(frz_device* dev, const void* const* buffers, int copies,
                     uint64_t bytes, uint32_t* sink, int iters, int graph,
                     double* us_per_launch);

/* Each pair's turns a position for a rotary base (src/core/kernels/rope/
 * rope.cpp:95-106): theta_k / 2 pi in f64, rounded once to f32. */
void frz_rope_turns(float base, int head_dim, float* turns);

/* ---- neuron pins (src/core/edit/edit.h:10-167) ---------------------------- */
/* An edit pins one neuron of a layer's feed-forward activation over the
 * steps [from, until) of a run (until 0xFFFFFFFF: to the end). */
enum frz_edit_kind { FRZ_EDIT_SET = 0, FRZ_EDIT_SCALE = 1, FRZ_EDIT_ZERO = 2 };
typedef struct frz_edit {
  uint32_t layer;
  uint32_t neuron;
  uint32_t kind;
  float value;
  uint32_t from;
  uint32_t until;
} frz_edit;
/* edit::EditError (src/core/edit/edit.h:131-141). */
enum frz_edit_error {
  FRZ_EDIT_OK = 0,
  FRZ_EDIT_ERR_KIND = 1,
  FRZ_EDIT_ERR_LAYER = 2,
  FRZ_EDIT_ERR_NEURON = 3,
  FRZ_EDIT_ERR_NOT_FINITE = 4,
  FRZ_EDIT_ERR_ZERO_VALUE = 5,
  FRZ_EDIT_ERR_RANGE = 6,
  FRZ_EDIT_ERR_OVERLAP = 7,
  FRZ_EDIT_ERR_TOO_MANY = 8
};
/* edit::check (src/core/edit/edit.cpp:105-134): the set's first fault and
 * the offending edit's index, or FRZ_EDIT_OK. */
int frz_edit_check(const frz_edit* edits, uint32_t count, uint32_t layers,
                   uint32_t ffn, uint32_t* offending);
/* Words of the table for `count` edits: 2 a layer + 5 an edit. */
uint32_t frz_edit_table_words(uint32_t count, uint32_t layers);
/* edit::table (src/core/edit/edit.cpp:136-161), ranges placed at origin
 * (origin 0 keeps them in steps). Precondition: frz_edit_check passed. */
int frz_edit_table(const frz_edit* edits, uint32_t count, uint32_t layers,
                   uint32_t origin, uint32_t* out_words);
/* edit::apply (src/core/edit/edit.cpp:93-103). */
float frz_edit_apply(uint32_t kind, float value, float neuron);

/* ---- the model and its steps (replaces Engine::finish_load +
 *      Program::build / Program::run, src/core/runtime/engine.cpp:342-394,
 *      src/core/kernels/program.h:338-387) ----------------------------------- */
typedef struct frz_model_config {
  int hidden;      /* 1152 */
  int ffn;         /* 6912 */
  int head_dim;    /* 256 */
  int query_heads; /* 4 */
  int kv_heads;    /* 1 */
  int layers;      /* 26 */
  int vocab;       /* 262144 */
  int window;      /* 512: a sliding layer's keys */
  int pattern;     /* 6: layer l is global when l % pattern == pattern - 1 */
  int context;     /* positions a global layer's cache holds */
  int local_slots; /* a sliding layer's ring: window + 512 + reserve */
  float rope_local;  /* 10,000 */
  float rope_global; /* 1,000,000 */
  float epsilon;     /* 1e-6 */
} frz_model_config;

/* Gemma-3-1B's shapes (src/core/arch/gemma3/gemma3.h:60-76). */
void frz_gemma3_1b_config(frz_model_config* out, int context);

/* Tensor roles a layer holds (src/core/arch/gemma3/gemma3.cpp:21-35), and the
 * two global tensors (layer -1). Matrices are Q4_0; norms are F32. */
enum frz_role {
  FRZ_ROLE_Q = 0,
  FRZ_ROLE_K = 1,
  FRZ_ROLE_V = 2,
  FRZ_ROLE_O = 3,
  FRZ_ROLE_GATE = 4,
  FRZ_ROLE_UP = 5,
  FRZ_ROLE_DOWN = 6,
  FRZ_ROLE_ATTN_NORM = 7,
  FRZ_ROLE_Q_NORM = 8,
  FRZ_ROLE_K_NORM = 9,
  FRZ_ROLE_POST_ATTN_NORM = 10,
  FRZ_ROLE_FFN_NORM = 11,
  FRZ_ROLE_POST_FFN_NORM = 12,
  FRZ_ROLE_EMBEDDING = 13,   /* layer -1: the tied token embedding / head */
  FRZ_ROLE_OUTPUT_NORM = 14  /* layer -1 */
};

/* Bytes of a tensor as a GGUF file holds it (Q4_0 blocks or F32). */
uint64_t frz_tensor_bytes(const frz_model_config* config, int role);

/* The seeded synthetic weights, host bytes of one tensor: Q4_0 blocks with
 * d = fp16(|N(0, 0.02)|) and codes uniform in 0..15; norm gains 1 +
 * 0.1 N(0, 1) (the file stores 1 + w). SplitMix64 streams keyed by (seed,
 * layer, role); normals by Box-Muller in f64. */
int frz_synth_tensor(const frz_model_config* config, uint64_t seed, int layer,
                     int role, void* out, uint64_t bytes);

/* ---- the capture store (src/core/capture/capture.h:43-75) ---------------
 * What the model used at the last position of the step that ends the prompt,
 * layer by layer, in one store of 32-bit words. Region 1: every layer's
 * neurons (the gated activation after the layer's pins, as the down product
 * reads it), in layer order. Region 2, layer by layer: the residual entering
 * the layer (the hidden row after its first norm's add; layer 0's is the
 * embedding row), what the attention block and the MLP block add to the
 * residual (their outputs after their post-norms), the query after QK-norm
 * and rope, the attention weights over the keys the query read, the
 * softmax statistics (m, l) of each head, and the readout: the top-64
 * (logit bits, token) pairs of the residual as the layer leaves it through
 * the final norm and the head (the last layer's: the step's own). */
typedef struct frz_capture_slot {
  uint32_t first;  /* word offset in the store */
  uint32_t width;  /* words */
} frz_capture_slot;
typedef struct frz_capture_slots {
  frz_capture_slot neurons, residual, attention_added, mlp_added, query,
      weights, stats, readout;
  uint32_t keys;   /* min(window, context): a head's weights */
  uint32_t query_heads;
  uint32_t window;
  uint32_t full_attention; /* window >= context */
} frz_capture_slots;
/* The store's words for a model of these shapes (0 for bad shapes), and
 * region 1's in *neuron_words when not null. */
uint64_t frz_capture_words(const frz_model_config* config,
                           uint64_t* neuron_words);
/* One layer's slots (capture.h: layout()). */
int frz_capture_layer(const frz_model_config* config, int layer,
                      frz_capture_slots* out);

/* ---- the tokenizer (src/core/tokenizer/tokenizer.h:124-247,
 *      bpe/sentencepiece_bpe.h:21-92) --------------------------------------
 * Gemma 3's SentencePiece BPE ("llama" in tokenizer.ggml.model), loaded
 * from a GGUF file's tokenizer.ggml.tokens, scores and token_type. Host
 * only: no device is needed. Encoding turns rendered text into ids: each
 * space becomes U+2581, control and user-defined tokens written as text
 * become their single ids (longest match from the left), every other
 * character its normal token or byte tokens, then adjacent normal symbols
 * merge, the highest-scoring token first, the leftmost on a tie. Nothing is
 * added: BOS is the template's text. Decoding gives each token's bytes (a
 * normal token's U+2581 as a space, a byte token's byte, any other token's
 * text as written). */
typedef struct frz_tokenizer frz_tokenizer;
enum frz_encode_error {
  FRZ_ENCODE_OK = 0,
  FRZ_ENCODE_INVALID_UTF8 = 1,
  FRZ_ENCODE_TOO_MANY_TOKENS = 2, /* more, at least, than max_tokens */
  FRZ_ENCODE_TOO_LONG = 3         /* past 512 KiB of normalized text */
};
#define FRZ_NO_TOKEN_LIMIT 0xFFFFFFFFu
/* EncodeResult (tokenizer.h:194-201). */
typedef struct frz_encode_result {
  int error; /* frz_encode_error */
  uint64_t least_tokens;
  uint64_t normalized_bytes;
  uint64_t raw_bytes;
} frz_encode_result;
/* Algorithm::load for the file's tokenizer; a refusal names its key. */
int frz_tokenizer_open(const char* gguf_path, frz_tokenizer** out);
void frz_tokenizer_free(frz_tokenizer* tokenizer);
uint32_t frz_tokenizer_size(const frz_tokenizer* tokenizer);
/* The longest token text, in bytes (tokenizer.h:70-72; 48 for Gemma 3). */
uint32_t frz_tokenizer_longest_cover(const frz_tokenizer* tokenizer);
/* A token's text as the file spells it, its type (1 normal, 2 unknown,
 * 3 control, 4 user-defined, 5 unused, 6 byte) and score. */
int frz_tokenizer_token(const frz_tokenizer* tokenizer, uint32_t id,
                        const char** text, uint32_t* bytes, int32_t* type,
                        float* score);
/* Tokenizer::encode: *count gets the ids' count and the first min(count,
 * cap) are written to ids; a refusal (result->error) writes none. */
int frz_tokenizer_encode(const frz_tokenizer* tokenizer, const char* text,
                         uint64_t bytes, uint32_t max_tokens, uint32_t* ids,
                         uint64_t cap, uint64_t* count,
                         frz_encode_result* result);
/* Tokenizer::decode of each id in turn: their bytes, *bytes of them (the
 * first cap written). */
int frz_tokenizer_decode(const frz_tokenizer* tokenizer, const uint32_t* ids,
                         uint32_t n, char* out, uint64_t cap, uint64_t* bytes);
/* A turn's input as text (detokenizer.h: texts): each id's text as a fresh
 * UTF-8 stream gives it, whole characters only, the last's with what ending
 * the stream gives (U+FFFD where bytes were pending); token i's text is
 * pool[offsets[i], offsets[i + 1]), n + 1 offsets. */
int frz_tokenizer_texts(const frz_tokenizer* tokenizer, const uint32_t* ids,
                        uint32_t n, char* pool, uint64_t cap,
                        uint64_t* pool_bytes, uint64_t* offsets);

typedef struct frz_model frz_model;

int frz_model_create(frz_device* dev, const frz_model_config* config,
                     frz_model** out);
void frz_model_destroy(frz_model* model);
/* One tensor from host bytes as a GGUF file holds it (Upload::write). */
int frz_model_set_tensor(frz_model* model, int layer, int role,
                         const void* data, uint64_t bytes);
/* The same in a given GGUF format (FRZ_FORMAT_*), as the pinned file mixes
 * them (src/core/formats/device_layout.h:64-66): the down matrices may be
 * Q4_0, Q4_1 or Q8_0, the embedding (and so the tied head) Q4_0 or Q8_0,
 * every other matrix Q4_0, the gains F32 (0). bytes = the role's blocks
 * times the format's block size. */
int frz_model_set_tensor_format(frz_model* model, int layer, int role,
                                int format, const void* data, uint64_t bytes);
/* Every tensor from frz_synth_tensor(seed). */
int frz_model_synthesize(frz_model* model, uint64_t seed);
/* The shapes the model was created with. */
int frz_model_get_config(const frz_model* model, frz_model_config* out);
/* One layer's launches of a one-token decode step at `position` (attention
 * norm and Q/K/V, rope and attention, O, feed-forward norm and gate-up with
 * the layer's pins, down), captured as one graph and replayed `iters` times,
 * timed with HIP events on the model's stream: the per-layer decode time of
 * the reference's one-layer decode configuration. The caches must hold the
 * context; the layer's slot at `position` is rewritten. */
int frz_model_time_layer(frz_model* model, int layer, uint32_t position,
                         uint32_t iters, double* us_per_layer);
/* Prompt tokens the last frz_generate (or frz_generate_variants) took from
 * the caches rather than computing them (the reference's Reply::reused,
 * runtime/runtime.h; the reuse rule of cache/prefix.h:87-94). */
uint32_t frz_model_reused(const frz_model* model);
/* The capture store on or off (off when created). While on, the step that
 * ends a prompt (a step asking for logits that is not a fed decode step)
 * writes every word of the store at its last row: Engine::inspect's and a
 * run's captures (src/core/capture/capture.h:15-34, :77-101), the store
 * laid out as frz_capture_layer says. It costs that step a head product,
 * a norm and a selection a layer for the readouts. */
int frz_model_set_capture(frz_model* model, int enabled);
/* The store's first `words` words, after the stream's work. */
int frz_model_read_capture(frz_model* model, uint32_t* out, uint64_t words);
/* The edit table, u32 words in the reference's layout (src/core/edit/
 * edit.h: per layer [first, count], then [neuron, kind, value bits, first
 * position, end position] per edit), used by every later step. */
int frz_model_set_edits(frz_model* model, const uint32_t* table,
                        uint32_t words);

/* How steps of several rows (prefill) compute their products. EXACT, the
 * default: in the reference's order of addition on the fp32 matrix cores,
 * bit for bit the reference's arithmetic. BF16: on the bf16 matrix cores
 * over split operands (each weight and activation as a pair hi + lo of
 * bf16), each product within about 2^-16 of the exact one, so logits agree
 * with the reference's within 1e-3 relative but not bit for bit; the caches
 * it writes then differ in their last bits too. Single-token decode steps
 * are EXACT either way. No counterpart in the reference (whose WGSL runs
 * fp32 only); switching forgets the cached prompt. */
enum frz_prefill_mode { FRZ_PREFILL_EXACT = 0, FRZ_PREFILL_BF16 = 1 };
int frz_model_set_prefill(frz_model* model, int mode);

/* Whether fed decode steps replay one captured HIP graph (1, the default)
 * or launch their kernels one by one (0: the same kernels, for tools that
 * trace launches). */
int frz_model_set_graphs(frz_model* model, int enabled);

/* One step of `tokens` (1 .. 512) token ids from `position`
 * (kernels::Step, src/core/kernels/interface.h:163-188). With logits, the
 * step also computes the last row's logits, selects and draws. Enqueued. */
int frz_model_step(frz_model* model, uint32_t position, uint32_t tokens,
                   const uint32_t* ids, int logits,
                   const frz_sampling* sampling);
/* `steps` fed decode steps, each from the last draw, after a step with
 * logits at `position` (the next token's position). Token i's id goes to
 * tokens_out[i] (and its failed flag to failed_out[i] when not null).
 * Replays one captured HIP graph per step; waits for the last. */
int frz_model_decode(frz_model* model, uint32_t position, uint32_t steps,
                     const frz_sampling* sampling, uint32_t* tokens_out,
                     uint32_t* failed_out);
/* Reads after a step (each waits for the device). */
int frz_model_read_logits(frz_model* model, float* out, uint32_t count);
int frz_model_read_record(frz_model* model, uint32_t record[4]);
int frz_model_read_candidates(frz_model* model, uint32_t out[128]);
int frz_model_read_hidden(frz_model* model, float* out, uint32_t rows);
int frz_model_read_cache(frz_model* model, int layer, int values,
                         uint16_t* out, uint64_t count);
/* Mean microseconds of each decode step over `steps` graph replays timed
 * with HIP events on the model's stream (the timed region of bench.py).
 * The steps rewrite the caches from `position` on, so the next
 * frz_generate computes its prompt afresh rather than reusing it. */
int frz_model_time_decode(frz_model* model, uint32_t position, uint32_t steps,
                          const frz_sampling* sampling, double* us_per_step);

/* ---- generation (replaces Engine::generate, src/core/runtime/engine.h:
 *      366-412, and the native tool's paired runs, tools/frizzle/main.cpp:
 *      53-55) ------------------------------------------------------------- */
/* Runs the prompt (prefill blocks of 512), then draws up to max_tokens
 * tokens with `edits` (the reference's edit table, placed at origin =
 * prompt_len - 1; null for none). Stops after a token in stop_ids. Returns
 * the tokens drawn in tokens_out and their count in *drawn. Reuses the cached
 * prefix of the model's last run where its tokens and placed edits agree
 * (src/core/cache/prefix.h:87-94). */
int frz_generate(frz_model* model, const uint32_t* prompt, uint32_t prompt_len,
                 const uint32_t* edit_table, uint32_t edit_words,
                 const frz_sampling* sampling, uint32_t max_tokens,
                 const uint32_t* stop_ids, uint32_t stops,
                 uint32_t* tokens_out, uint32_t* drawn);
/* Many continuations of one prompt at once: an original and steered
 * variants of it from one seed, decoded as one batch. The reference runs
 * such replies one at a time (the paired runs of tools/frizzle/main.cpp:
 * 53-55 through runtime/engine.h:60-139); this runs them together. Variant
 * v runs under its own edit table,
 * edit_tables + v * table_words words in frz_edit_table's layout with
 * ranges in steps, placed at the prompt's last position as frz_generate
 * places one; all share `sampling`. The prompt but its last token is
 * computed once, through the model's own caches (and reused as frz_generate
 * reuses it); each variant then gets a copy of those caches, and every step
 * runs one token of every variant through each product together. Variant
 * v's tokens are the ones frz_generate gives for its table alone, bit for
 * bit, ending likewise at a stop token or a failed draw:
 * tokens_out[v * max_tokens ...], drawn_out[v] of them. residuals_out, when
 * not null, receives [max_tokens][layers][variants][hidden] floats: at each
 * step, the residual entering each layer (the hidden row after the add of
 * the layer's first norm; layer 0's is the embedding row), as the capture
 * store defines it (src/core/capture/capture.h:15-17). 1 to 64 variants. */
int frz_generate_variants(frz_model* model, const uint32_t* prompt,
                          uint32_t prompt_len, uint32_t variants,
                          const uint32_t* edit_tables, uint32_t table_words,
                          const frz_sampling* sampling, uint32_t max_tokens,
                          const uint32_t* stop_ids, uint32_t stops,
                          uint32_t* tokens_out, uint32_t* drawn_out,
                          float* residuals_out);

/* ---- GGUF files (replaces the reference's gguf::read_index and the
 *      Gemma 3 load, src/core/gguf/reader.h:12-107, index.h,
 *      src/core/arch/gemma3/gemma3.cpp:21-95, describe.cpp:205-290) ------- */

/* The ways reading a file's index can fail, each a named rule of the file
 * (the reference's ReadError, src/core/gguf/types.h:237-265). */
enum frz_gguf_error {
  FRZ_GGUF_OK = 0,
  FRZ_GGUF_NEED_MORE_BYTES = 1,   /* inside the file, not yet supplied */
  FRZ_GGUF_SHORT_READ = 2,        /* the file ends before this field */
  FRZ_GGUF_BAD_MAGIC = 3,
  FRZ_GGUF_UNSUPPORTED_VERSION = 4,
  FRZ_GGUF_COUNT_TOO_LARGE = 5,   /* over 2^20 tensors or metadata entries */
  FRZ_GGUF_STRING_TOO_LONG = 6,   /* over 2^20 bytes */
  FRZ_GGUF_ARRAY_TOO_LONG = 7,    /* over 2^24 elements */
  FRZ_GGUF_UNKNOWN_VALUE_TYPE = 8,
  FRZ_GGUF_UNKNOWN_TENSOR_TYPE = 9,
  FRZ_GGUF_ROW_NOT_WHOLE_BLOCKS = 10,
  FRZ_GGUF_TOO_MANY_DIMENSIONS = 11,
  FRZ_GGUF_NEGATIVE_DIMENSION = 12,
  FRZ_GGUF_ELEMENT_COUNT_OVERFLOW = 13,
  FRZ_GGUF_OFFSET_OVERFLOW = 14,
  FRZ_GGUF_TENSOR_DATA_OUT_OF_BOUNDS = 15,
  FRZ_GGUF_DUPLICATE_TENSOR_NAME = 16,
  FRZ_GGUF_TENSOR_NAME_TOO_LONG = 17, /* over 64 bytes */
  FRZ_GGUF_MISALIGNED_TENSOR_DATA = 18,
  FRZ_GGUF_OVERLAPPING_TENSOR_DATA = 19,
  FRZ_GGUF_BAD_ALIGNMENT = 20,    /* general.alignment: not a power-of-two uint32 */
  FRZ_GGUF_EMPTY_KEY = 21,
  FRZ_GGUF_DUPLICATE_METADATA_KEY = 22,
  FRZ_GGUF_NESTED_ARRAY = 23
};

typedef struct frz_gguf frz_gguf;

/* One tensor of the index: GGUF's format number, its extents (ne0 first,
 * unused ones 1), and its absolute byte range in the file. */
typedef struct frz_gguf_tensor {
  char name[65];
  uint32_t type;
  uint32_t dimensions;
  uint64_t shape[4];
  uint64_t elements;
  uint64_t offset;
  uint64_t bytes;
} frz_gguf_tensor;

/* Reads the index of a file of `file_size` bytes whose first `resident`
 * bytes are at `front`; tensor data is never read. Returns a
 * frz_gguf_error. On FRZ_GGUF_OK, *out is a new index (frz_gguf_free); on
 * FRZ_GGUF_NEED_MORE_BYTES, *bytes_needed is the length of front, from byte
 * 0, the read needed; *out is untouched unless the read succeeds. -1 for a
 * null `out`, or a null `front` with resident bytes. */
int frz_gguf_read(const void* front, uint64_t resident, uint64_t file_size,
                  frz_gguf** out, uint64_t* bytes_needed);
/* The same from a file's path, reading its front as the index asks.
 * Returns a frz_gguf_error, or -1 when the file cannot be opened or read. */
int frz_gguf_open(const char* path, frz_gguf** out);
void frz_gguf_free(frz_gguf* index);
const char* frz_gguf_error_text(int error);
/* A format's name and block (elements, bytes); FRZ_ERR_ARGUMENT for a number
 * GGUF does not define. */
int frz_gguf_format(uint32_t type, const char** name, uint32_t* block_elements,
                    uint32_t* block_bytes);

uint64_t frz_gguf_tensor_count(const frz_gguf* index);
int frz_gguf_tensor_at(const frz_gguf* index, uint64_t i, frz_gguf_tensor* out);
/* FRZ_ERR_ARGUMENT when no tensor has the name. */
int frz_gguf_find(const frz_gguf* index, const char* name, frz_gguf_tensor* out);
uint64_t frz_gguf_metadata_count(const frz_gguf* index);
/* Metadata by key. An integer of any width that fits, a FLOAT32/FLOAT64
 * as float, a string (length without the terminator; the text is cut to
 * cap - 1 bytes and terminated), an array's element type and count.
 * FRZ_ERR_ARGUMENT when the key is absent or holds another kind. */
int frz_gguf_get_u32(const frz_gguf* index, const char* key, uint32_t* out);
int frz_gguf_get_f32(const frz_gguf* index, const char* key, float* out);
int frz_gguf_get_string(const frz_gguf* index, const char* key, char* buf,
                        uint64_t cap, uint64_t* length);
int frz_gguf_get_array(const frz_gguf* index, const char* key,
                       uint32_t* element_type, uint64_t* count);

/* A Gemma 3 model's shapes from its metadata and its token embedding
 * (describe.cpp:205-290, gemma3.cpp:44-95): gemma3.block_count,
 * embedding_length, feed_forward_length, attention.head_count,
 * attention.head_count_kv, attention.key_length (default width / heads),
 * attention.layer_norm_rms_epsilon, rope.freq_base, rope.freq_base_swa
 * (default 10,000), attention.sliding_window, sliding_window_pattern
 * (default 6); the vocabulary is token_embd.weight's second extent.
 * `context` positions for the global caches (0: 8,192). */
int frz_gemma3_config_from_gguf(const frz_gguf* index, int context,
                                frz_model_config* out);
/* Loads every tensor of a Gemma 3 GGUF file into a model created with that
 * file's shapes: blk.N.{attn_q,attn_k,attn_v,attn_output,ffn_gate,ffn_up,
 * ffn_down}.weight (Q4_0), blk.N.{attn_norm,attn_q_norm,attn_k_norm,
 * post_attention_norm,ffn_norm,post_ffw_norm}.weight (F32),
 * token_embd.weight (Q4_0, tied head) and output_norm.weight (F32).
 * FRZ_ERR_ARGUMENT, naming the tensor, for a missing tensor, a shape that
 * is not the model's, a format this backend does not run, or an untied
 * output.weight. */
int frz_model_load_gguf(frz_model* model, const char* path);

/* ---- the residency plan (replaces residency::plan_residency,
 *      src/core/residency/plan.h:14-326, under policy::LoadPolicy,
 *      src/core/policy/policy.h:23-76) -----------------------------------
 * Where every weight, each layer's KV cache and every working buffer lies
 * on the device, and the context offered: a pure function of a Gemma 3
 * file's index, the device's limits and the load policy (no device, no
 * I/O). Three pools never share a buffer; every range starts at a multiple
 * of the alignment and is its bytes rounded up to 4, at most min(binding,
 * buffer) long. A weight is cut into pieces of whole rows in file order; a
 * layer's Q, K, V and its gate, up form a group when they share a format and
 * an input width and their span fits one range in one buffer. Each working
 * buffer (the decoder's 18, graph.cpp:132-198) is a buffer of its own. A
 * sliding layer's cache is a ring of window + 512 + rollback_reserve slots,
 * a full-attention layer's the context offered: the largest from
 * min(512, trained) to the trained context (gemma3.context_length) whose
 * cache fits beside the weights and working buffers within the budget. */
typedef struct frz_plan_limits {
  uint64_t max_buffer_size;
  uint64_t max_storage_binding_size;
  uint32_t storage_offset_alignment; /* a power of two */
} frz_plan_limits;
/* LoadPolicy with its F16 cache: the bytes the plan may place, and the
 * tokens a sliding layer's ring keeps beyond one step for rollback. */
typedef struct frz_load_policy {
  uint64_t memory_budget;
  uint32_t rollback_reserve;
} frz_load_policy;
/* policy.h's defaults: 2 GiB, 4,096. */
void frz_load_policy_default(frz_load_policy* out);
/* PlanError (plan.h:305-319), plus a file that describes no Gemma 3 model. */
enum frz_plan_error {
  FRZ_PLAN_OK = 0,
  FRZ_PLAN_EXCEEDS_BUDGET = 1,       /* summary->total_bytes: what 512 needs */
  FRZ_PLAN_ROW_EXCEEDS_BINDING = 2,  /* subject: the tensor */
  FRZ_PLAN_SCRATCH_EXCEEDS_BINDING = 3, /* subject: the working buffer */
  FRZ_PLAN_OVERFLOW = 4,
  FRZ_PLAN_NOT_DESCRIBED = 5         /* subject: the metadata key or tensor */
};
enum frz_pool { FRZ_POOL_WEIGHTS = 0, FRZ_POOL_CACHE = 1, FRZ_POOL_SCRATCH = 2 };
typedef struct frz_range {
  uint32_t buffer;
  uint64_t offset;
  uint64_t length;
} frz_range;
/* A weight piece: its range and the rows of the tensor it holds. */
typedef struct frz_piece {
  frz_range range;
  uint64_t first_row;
  uint64_t rows;
} frz_piece;
typedef struct frz_plan_summary {
  uint32_t buffers, tensors, pieces, groups, layers, scratch;
  uint32_t partial_rows;
  uint32_t context_offered;
  uint32_t trained_context;
  uint64_t weight_bytes, cache_bytes, scratch_bytes, total_bytes;
} frz_plan_summary;
typedef struct frz_plan frz_plan;
/* Plans the Gemma 3 model of `index`. Returns a frz_plan_error; on
 * FRZ_PLAN_OK *out is a new plan (frz_plan_free). `subject` (when not null)
 * receives the refusal's subject, cut to subject_cap - 1 bytes. */
int frz_plan_gemma3(const frz_gguf* index, const frz_plan_limits* limits,
                    const frz_load_policy* policy, frz_plan** out,
                    frz_plan_summary* summary, char* subject, size_t subject_cap);
void frz_plan_free(frz_plan* plan);
const char* frz_plan_error_text(int error);
int frz_plan_summarize(const frz_plan* plan, frz_plan_summary* out);
/* A tensor's GGUF format as the plan placed it. */
int frz_plan_format(const frz_plan* plan, uint64_t tensor, uint32_t* format);
/* The model's shapes, its context the context offered and its sliding
 * rings the plan's. */
int frz_plan_config(const frz_plan* plan, frz_model_config* out);
int frz_plan_buffer(const frz_plan* plan, uint32_t index, int* pool, uint64_t* size);
/* Tensor `tensor` of the index (index order): *pieces its piece count, and
 * piece `piece` into *out when out is not null. */
int frz_plan_tensor(const frz_plan* plan, uint64_t tensor, uint32_t piece, frz_piece* out,
                    uint32_t* pieces);
/* Group i: its members (tensor indices, output order), count and span. */
int frz_plan_group(const frz_plan* plan, uint32_t index, uint64_t members[3],
                   uint32_t* count, frz_range* span);
int frz_plan_cache(const frz_plan* plan, uint32_t layer, frz_range* keys,
                   frz_range* values, uint32_t* slots);
/* A working buffer by its purpose ("hidden", "normed", ..., "captures"). */
int frz_plan_scratch(const frz_plan* plan, const char* purpose, frz_range* out);
/* The tensor index of a layer's role (layer -1: the embedding or the
 * output norm). */
int frz_plan_role(const frz_plan* plan, int layer, int role, uint64_t* tensor);
/* Limits this device grants a plan: buffers and bindings as large as its
 * memory, ranges aligned to 256 bytes (every tensor stays in one piece). */
int frz_device_plan_limits(frz_device* dev, frz_plan_limits* out);
/* A model created from a plan (replaces Engine::begin_load's Upload::begin
 * over the plan, src/core/runtime/engine.cpp:575, upload.h:276): one
 * allocation for each planned buffer; every weight, norm gain and layer
 * cache at its planned range, in the device layout (a layer's Q, K and V
 * read as one product over the three members the plan grouped); the
 * context the plan offered and its rings. The working buffers the plan
 * names that this backend reads as they are (hidden, normed, attention,
 * output, activation, logits, candidates, sampled, edit_table, captures)
 * are the planned ones; the backend's own (the fused Q/K/V rows, a second
 * hidden row, the attention partials of every chunk, the selection's
 * scratch, the token log) are allocated beside them. Every weight must be
 * one piece (frz_device_plan_limits keeps them so), Q, K and V Q4_0 with
 * K = 1,152. Tensors are then set as for any model (frz_model_set_tensor*,
 * frz_model_load_gguf), each in the format the plan placed it in. */
int frz_model_create_planned(frz_device* dev, const frz_plan* plan, frz_model** out);
/* The planned buffer `index` of a model created from a plan: its device
 * address and size (for a caller that writes a tensor's bytes itself). */
int frz_model_planned_buffer(const frz_model* model, uint32_t index, void** dev_ptr,
                             uint64_t* size);

/* ---- the program (replaces kernels::Program, src/core/kernels/program.h:
 *      264-402, over kernels::Launch, interface.h:320-363, reported in order
 *      as kernels::Order does, order.h:68-104) ------------------------------
 * A graph's launches, as graph::Builder emits them for Gemma 3
 * (src/core/graph/graph.cpp:290-470), each described as the reference's
 * Launch with its WGSL named by a kernel number instead of its text. The
 * program recognises the Gemma 3 graph in them (every stage in the graph's
 * order, named by its role and layer as graph.h names them, and bound to
 * the plan's tensors, caches and working buffers) and runs each step
 * through this backend's fused kernels; anything else is refused, Build,
 * naming the launch. */
enum frz_kernel {
  FRZ_KERNEL_GATHER = 0,            /* kernels/gather/gather.wgsl */
  FRZ_KERNEL_NORM = 1,              /* kernels/norm/norm.wgsl */
  FRZ_KERNEL_MATMUL = 2,            /* kernels/matmul/matmul.wgsl, any entry point */
  FRZ_KERNEL_ROPE = 3,              /* kernels/rope/rope.wgsl with rope_cache.wgsl */
  FRZ_KERNEL_ATTENTION = 4,         /* kernels/attention/attention.wgsl main */
  FRZ_KERNEL_ATTENTION_COMBINE = 5, /* attention.wgsl combine */
  FRZ_KERNEL_EDIT = 6,              /* edit/edit.wgsl */
  FRZ_KERNEL_TOPK = 7,              /* kernels/topk/topk.wgsl, either pass */
  FRZ_KERNEL_DRAW = 8,              /* sampler/draw.wgsl */
  FRZ_KERNEL_CAPTURE = 9,           /* capture/capture.wgsl: a copy or a readout */
  FRZ_KERNEL_CAPTURE_WEIGHTS = 10   /* capture/weights.wgsl */
};
enum frz_rows { FRZ_ROWS_EVERY_TOKEN = 0, FRZ_ROWS_LAST_TOKEN = 1, FRZ_ROWS_PROMPT_END = 2 };
enum frz_key_split {
  FRZ_KEY_SPLIT_NONE = 0,
  FRZ_KEY_SPLIT_PER_CHUNK = 1,
  FRZ_KEY_SPLIT_WHEN_SPLIT = 2
};
#define FRZ_NO_LAYER 0xFFFFFFFFu
/* A bound range of one of the plan's buffers (kernels::Binding). */
typedef struct frz_binding {
  uint32_t buffer;
  uint64_t offset;
  uint64_t size;
} frz_binding;
/* kernels::Override (interface.h:310-314): a WGSL override constant and its
 * value. This backend's kernels are compiled for the Gemma 3 shapes and take
 * none: a build makes Program::build's checks of a launch's overrides
 * (program.cpp:432-444: "workgroup_size" and "last_token" are the program's
 * to set, and no name is given twice), then ignores them by name. */
typedef struct frz_override {
  const char* name;
  double value;
} frz_override;
/* kernels::Launch. `role` and `layer` are the graph's names (graph.h). */
typedef struct frz_launch {
  int kernel;              /* frz_kernel */
  const char* entry_point; /* the WGSL entry point, or null for "main" */
  int format;              /* GGUF format of the weights it unpacks, or -1 */
  int pack_format;         /* the format it packs (the cache's), or -1 */
  const void* constants;
  uint32_t constants_bytes; /* at most 768 */
  const frz_binding* bindings;
  uint32_t binding_count;
  uint32_t invocations_per_row;
  uint32_t workgroup_size;
  int rows;                /* frz_rows */
  uint32_t rows_per_tile;  /* 0: a launch over rows */
  int key_split;           /* frz_key_split */
  uint32_t window;
  uint32_t partial_rows;
  uint32_t tokens_least, tokens_most; /* the steps it runs in, by token count */
  const char* role;
  uint32_t layer;          /* FRZ_NO_LAYER for the embedding and the output */
  const frz_override* overrides; /* Launch::overrides, interface.h:335 */
  uint32_t override_count;
} frz_launch;
/* kernels::Step: the 64-byte head (sampler::apply's settings and seed) and
 * the step's token ids. */
typedef struct frz_step_record {
  uint32_t position;
  uint32_t tokens;     /* 1 .. 512 */
  uint32_t logits;     /* 1: the last token's logits are drawn from */
  uint32_t fed;        /* 1: one token, the last step's draw */
  uint32_t seed[2];
  uint32_t top_k;
  float temperature;
  float top_p;
  float min_p;
  float log_min_p;
  uint32_t padding[5];
  uint32_t ids[512];
} frz_step_record;
/* kernels::RunInput: bytes written into a range of one of the plan's
 * buffers before the step (to.size bytes from `bytes`). */
typedef struct frz_run_input {
  frz_binding to;
  const void* bytes;
} frz_run_input;
/* kernels::StepCallback: `readback` (the draw's 16-byte record for a step
 * that asked for logits) and `message` are valid only during the call. */
typedef void (*frz_step_callback)(int status, const char* message, const void* readback,
                                  uint32_t readback_bytes, void* userdata);
typedef struct frz_program frz_program;

/* The build's checks without a device (Program::build's refusals,
 * program.h:29-41, then the Gemma 3 graph's recognition): FRZ_OK, or
 * FRZ_ERR_BUILD with the message naming the launch. Pure. */
int frz_program_check(const frz_plan* plan, const frz_launch* launches, uint32_t count,
                      const frz_binding* readback, char* message, size_t message_cap);
/* Program::build over a model created from `plan` (the upload whose buffers
 * the bindings index; it must outlive the program). The program turns the
 * model's capture store on, as the graph's capture launches write it. */
int frz_program_build(frz_model* upload, const frz_plan* plan, const frz_launch* launches,
                      uint32_t count, const frz_binding* readback, frz_program** out,
                      char* message, size_t message_cap);
/* Program::run: at most two steps outstanding. Refused at once, FRZ_ERR_STEP
 * through `done` before this returns (and not numbered): a third step while
 * two are outstanding, a step of 0 or more than 512 tokens, and any step
 * once the device is lost (FRZ_ERR_DEVICE_LOST). Failed, FRZ_ERR_STEP, with
 * nothing run, reported in order: a step past the context, or an input
 * outside its buffer or not of whole words. Otherwise `done` is called by
 * frz_poll once the step has finished. */
int frz_program_run(frz_program* program, const frz_step_record* step,
                    const frz_run_input* inputs, uint32_t input_count,
                    frz_step_callback done, void* userdata);
/* Calls the callbacks of the steps that have settled, in the order they
 * were run (a later one waits for an earlier), on the calling thread. With
 * `wait`, first waits for the oldest outstanding step. The number of
 * callbacks made. */
int frz_poll(frz_program* program, int wait);
uint32_t frz_program_outstanding(const frz_program* program);
/* Reports every outstanding step FRZ_ERR_CANCELLED, in run order, once the
 * device has finished it (its results are not reported); the program stays
 * usable (the runtime's cancel, runtime.h:49-56). */
int frz_program_cancel(frz_program* program);
/* Destroys the program; outstanding steps are reported FRZ_ERR_CANCELLED. */
void frz_program_destroy(frz_program* program);
/* A host-side stand-in for the device reporting itself lost (no device
 * fault is made): steps settling from now on are reported
 * FRZ_ERR_DEVICE_LOST and new ones refused so. For tests of the failure
 * path; a real loss (a HIP error on the stream) takes the same path. */
int frz_program_mark_lost(frz_program* program);

/* ---- profiled steps ------------------------------------------------------
 * A step run as usual, launch by launch (no captured graph), with a HIP
 * event recorded on the stream before each launch and after the last. Each
 * launch is named by what it does in the model, as the reference's graph
 * names its launches (kernels::Launch::role and ::layer, interface.h:356-362;
 * the names of graph/graph.h:99-106): "embed", "attention.norm",
 * "attention.qkv", "attention.rope", "attention.scores",
 * "attention.combine", "attention.output", "ffn.norm", "ffn.gate_up",
 * "ffn.edit", "ffn.down", "output.norm", "output.head", "output.select",
 * "output.draw", and the capture store's "attention.capture",
 * "attention.weights", "ffn.capture", "readout", "output.readout". A launch of this backend
 * that runs several of the graph's roles (a product with its norm in its
 * prologue) names them all, joined by "+". A step's results are those of an
 * unprofiled one. */
typedef struct frz_launch_time {
  char role[96];
  uint32_t layer;        /* FRZ_NO_LAYER for the embedding and the output */
  uint32_t graph_index;  /* a program's: the graph's last launch it runs; else ~0 */
  double microseconds;   /* from the event before it to the one after it */
} frz_launch_time;
/* frz_model_step, profiled (no reference counterpart at the model level: a
 * diagnostic entry, as Program::run_profiled is the program's). `count` gets
 * the step's launches; at most `cap` are written to `out`. */
int frz_model_profile_step(frz_model* model, uint32_t position, uint32_t tokens,
                           const uint32_t* ids, int logits, const frz_sampling* sampling,
                           frz_launch_time* out, uint32_t cap, uint32_t* count);
/* One fed decode step (the last step's draw at `position`, as one step of
 * frz_model_decode), profiled; *token gets its draw. */
int frz_model_profile_decode(frz_model* model, uint32_t position, const frz_sampling* sampling,
                             frz_launch_time* out, uint32_t cap, uint32_t* count,
                             uint32_t* token);
/* Program::run_profiled's Timestamps (program.h:344-357): nanoseconds, the
 * step's first event at 0 (begin_ns), its last at end_ns, and the end of each
 * of this backend's launches by the index, in the graph, of the last of the
 * graph's launches it runs. Valid only during the callback. */
typedef struct frz_profile_times {
  uint64_t begin_ns;
  uint64_t end_ns;
  const uint32_t* launch_index;
  const uint64_t* launch_end_ns;
  const frz_launch_time* launches;  /* the same launches, named and timed */
  uint32_t launch_count;
} frz_profile_times;
typedef void (*frz_profile_callback)(int status, const char* message, const void* readback,
                                     uint32_t readback_bytes, const frz_profile_times* times,
                                     void* userdata);
/* Program::run_profiled (program.h:359-365): runs one step as
 * frz_program_run does, timed; `done` is called by frz_poll in run order,
 * with zero times for a step refused or failed. `launches` must be the
 * graph's whole count (frz_program_launch_count): this backend's launches
 * each run several of the graph's, so it runs no prefix of a step. Refused
 * at once, FRZ_ERR_STEP: a prefix, a step beside an unprofiled one
 * outstanding, and frz_program_run's refusals. */
int frz_program_run_profiled(frz_program* program, const frz_step_record* step,
                             const frz_run_input* inputs, uint32_t input_count,
                             uint32_t launches, frz_profile_callback done, void* userdata);
/* Program::launch_count (program.h:367-368): the graph's launches. */
uint32_t frz_program_launch_count(const frz_program* program);
/* Program::can_profile (program.h:370-372): 1 (HIP events time every
 * launch on this backend). */
int frz_program_can_profile(const frz_program* program);

#ifdef __cplusplus
}
#endif

#endif /* FRIZZLE_HIP_H */
