/* lrm_hip.h — the C ABI of liblrm_hip.so, the MI355X (gfx950) HIP device and Qwen3 executor for enderPeer/rosylnalive.
 *
 * Every function returns an int status (LRM_OK = 0) unless stated; on failure lrm_last_error() holds a message on the
 * calling thread. LRM_E_CONTRACT is the reference's GpuContractException (src/Lrm.Gpu.Core/Errors.fs:7-13), raised by
 * the same host-side checks before any device work; LRM_E_HIP is a device or HIP API failure (the reference's
 * backend-specific exception). Calls on one device come from one thread at a time (src/Lrm.Gpu.Core/Backend.fs:138).
 * No PyTorch or HIP types cross this boundary: plain pointers, sizes and opaque handles only.
 *
 * Each declaration names the reference interface it replaces (file:line in enderPeer/rosylnalive).
 */
#ifndef LRM_HIP_H
#define LRM_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LRM_OK 0
#define LRM_E_CONTRACT 1 /* GpuContractException */
#define LRM_E_HIP 2      /* device lost, HIP API failure */
#define LRM_E_ARG 3      /* invalid argument to the executor or a helper */
#define LRM_E_INTERNAL 4
#define LRM_E_RANGE 5 /* a value the fast path stores as fp16 (activation, K/V cache entry) became inf or NaN */
#define LRM_E_FORMAT 6    /* SafetensorsFormatException (src/Lrm.Tensor/Safetensors.fs:15-17) */
#define LRM_E_INTEGRITY 7 /* IntegrityException (Safetensors.fs:20-34): size or SHA-256 differs from the pinned one */
#define LRM_E_DATA 8      /* InvalidDataException (src/Lrm.Tokenizer/TokenizerJson.fs:24-25): tokenizer.json refused */

#define LRM_ABI_VERSION 1

/* Message of the last failure on this thread (never NULL). */
const char *lrm_last_error(void);
int lrm_abi_version(void);

/* ======================================================================== contract helpers (host only, no GPU)
 * The shared checks of Lrm.Gpu.Core, exported so a host that builds its own tables (the F# side) and tests can use the
 * exact rules the device enforces. */

/* Kernels.all / catalog.json (src/Lrm.Gpu.Core/Kernels.g.fs:27-285): ids 0..13 are the reference catalog, 14.. are
 * this backend's appended fast-path kernels. kind: 1 token, 2 u32, 3 i32, 4 f32; access: 1 read, 2 write, 3 readwrite,
 * 4 meta; dtype_mask: bit (1 << DType code). */
int lrm_catalog_count(void);
int lrm_catalog_find(const char *name); /* id, or -1 */
int lrm_catalog_kernel(uint32_t id, char *name, int name_cap, uint32_t threads[3], int *linear, int *field_count);
int lrm_catalog_field(uint32_t id, int field, char *name, int name_cap, int *kind, int *access, uint32_t *dtype_mask);

/* Grid.physical (src/Lrm.Gpu.Core/ArgBlock.fs:368-387): folds a linear grid above 65,535 groups. */
int lrm_grid_physical(int linear, int64_t x, int64_t y, int64_t z, uint32_t out[3]);

/* TensorRow.create and debugIdOf (src/Lrm.Gpu.Core/TensorTable.fs:60-230). */
int lrm_tensor_row(int slot, uint64_t byte_offset, uint32_t dtype, const uint32_t *dims, int rank, uint32_t flags,
                   const char *name, uint32_t out_words[16]);
uint32_t lrm_debug_id(const char *name);

/* HeapPlanner (src/Lrm.Gpu.Core/HeapLayout.fs:433-525). */
typedef struct lrm_planner lrm_planner;
int lrm_planner_create(uint64_t page_bytes, lrm_planner **out);
int lrm_planner_allocate(lrm_planner *p, uint32_t arena, uint64_t bytes, int32_t *page_index, uint64_t *offset);
int lrm_planner_build(lrm_planner *p, uint32_t *arenas, uint64_t *page_bytes, int capacity, int *pages);
void lrm_planner_destroy(lrm_planner *p);

/* TensorTable and SealedTable (src/Lrm.Gpu.Core/TensorTable.fs:378-474), over a layout given as HeapLayout.ofPages
 * (src/Lrm.Gpu.Core/HeapLayout.fs:302-420): pages[i] = (arena code, bytes). */
typedef struct lrm_table lrm_table;
int lrm_table_create(const uint32_t *arenas, const uint64_t *page_bytes, int pages, lrm_table **out);
int lrm_table_add(lrm_table *t, const char *name, int slot, uint64_t byte_offset, uint32_t dtype, const uint32_t *dims,
                  int rank, uint32_t flags, uint32_t *token);
int lrm_table_add_view(lrm_table *t, const char *name, uint32_t source, const uint32_t *dims, int rank,
                       uint64_t element_offset, uint32_t *token);
int lrm_table_seal(lrm_table *t, uint8_t *image_out /* 1 MiB */);
void lrm_table_destroy(lrm_table *t);

/* Dispatch.prepare (src/Lrm.Gpu.Core/Dispatch.fs:149-173) against a sealed image and layout: checks the block and
 * writes the dispatched words (word 0 = physical x), the logical grid and the physical grid. */
int lrm_prepare(const uint8_t *table_image, const uint32_t *arenas, const uint64_t *page_bytes, int pages,
                uint32_t kernel, const uint32_t in_words[32], uint32_t out_words[32], int64_t grid[3],
                uint32_t physical[3]);

/* ======================================================================== the device
 * IGpuBackendProvider.Enumerate / Create (src/Lrm.Gpu.Core/Backend.fs:156-161), DeviceInfo (Backend.fs:9-31). */
typedef struct lrm_hip_device_info {
    int32_t index;
    char name[128];
    char arch[64]; /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    uint32_t vendor_id; /* 0x1002 */
    uint32_t pci_device_id;
    char pci_bus[32];
    char driver[64];
    int64_t memory_bytes;
    int32_t compute_units;
} lrm_hip_device_info;

int lrm_hip_enumerate(lrm_hip_device_info *infos, int capacity, int *count);

typedef struct lrm_hip_device lrm_hip_device;
#define LRM_HIP_TIME_DISPATCHES 1u /* DeviceOptions.TimeDispatches (Backend.fs:38-55) */
int lrm_hip_create(int index, uint32_t flags, lrm_hip_device **out);
int lrm_hip_destroy(lrm_hip_device *d); /* IDisposable: waits for outstanding work */
int lrm_hip_info(lrm_hip_device *d, lrm_hip_device_info *out);

/* IGpuHeap (Backend.fs:111-122): CreateHeap once, WriteTable once before the first dispatch, Upload/Download wait for
 * all submitted work first. */
int lrm_hip_create_heap(lrm_hip_device *d, const uint32_t *arenas, const uint64_t *page_bytes, int pages);
int lrm_hip_write_table(lrm_hip_device *d, const void *image, uint64_t bytes);
int lrm_hip_upload(lrm_hip_device *d, int slot, uint64_t offset, const void *src, uint64_t bytes);
int lrm_hip_download(lrm_hip_device *d, int slot, uint64_t offset, void *dst, uint64_t bytes);

/* IGpuBackend.LoadKernels / IKernelSet (Backend.fs:104-108,144-147): the gfx950 code objects are part of this
 * library. Loads the reference kernel set (catalog ids 0-13, Kernels.g.fs:27-285), which keeps the BatchInvariance
 * contract (docs/contracts/batch-invariance.md:7-12). The shader-set hash, which fills ExecutionClass.ShaderSetHash
 * (ExecutionClass.fs:58), is the SHA-256 of the set's name and the library file's SHA-256. Runs the fp32 denormal
 * probe (Backend.fs:457-547): mode 1 preserve, 2 flush, 3 mixed. */
int lrm_hip_load_kernels(lrm_hip_device *d, uint8_t shader_set_hash[32]);
/* An extension of LoadKernels: the set to load, once per backend. LRM_HIP_KERNELS_FAST is every id (0-40, the
 * appended fast path included) under its own shader-set hash, so its results form their own ExecutionClass: it only
 * claims that the same work on the same inputs gives the same bits (the row count chooses its k-split and attention
 * splits; its prefill and decode kernels sum in different orders), and no bit-identity claim crosses the two sets. */
#define LRM_HIP_KERNELS_REFERENCE 0u
#define LRM_HIP_KERNELS_FAST 1u
int lrm_hip_load_kernel_set(lrm_hip_device *d, uint32_t set, uint8_t shader_set_hash[32]);
int lrm_hip_contains(lrm_hip_device *d, uint32_t kernel); /* 1 or 0 */
/* Diagnostics, no counterpart in the reference: the per-workgroup stamps of the prefill GEMMs' direct-to-LDS loop
 * recorded by the stage-timing build of this library (python -m rosylnalive_amd.build --stamps), for the last launch
 * of each GEMM kind (kind = epilogue: 0 f32, 1 residual, 2 SwiGLU, 3 q|k|v, 4 k-split partials). 32 words per
 * workgroup (linear block id): word 0 = (XCC_ID << 32) | HW_ID, 1 start, 2 + kt tile kt landed, 30 main loop end, 31
 * epilogue end, in 100 MHz constant-clock ticks. The shipped build records nothing and returns LRM_E_ARG. */
int lrm_hip_debug_gemm_stamps(lrm_hip_device *d, uint32_t kind, uint64_t *dst, uint64_t words);
int lrm_hip_denormal_probe(lrm_hip_device *d, int *mode, uint32_t results[7]);

/* ICommandList (Backend.fs:125-136) and IGpuBackend.Begin/Submit/Wait (Backend.fs:148-153). A list created with
 * reusable = 1 is an extension for replay: it is captured into a HIP graph at its first submission and every
 * submission (with `repeat` >= 1) replays it; it may not hold timers. One-shot lists are closed by Submit. */
typedef struct lrm_hip_list lrm_hip_list;
int lrm_hip_begin(lrm_hip_device *d, int reusable, lrm_hip_list **out);
int lrm_hip_dispatch(lrm_hip_list *l, uint32_t kernel, const uint32_t words[32]);
/* ICommandList.Dispatch for work that may overlap what follows (an extension; the reference's ordering rule,
 * docs/contracts/gpu-backend.md:58-64, lets dispatches not separated by Barrier overlap, while lrm_hip_dispatch runs
 * each dispatch after the previous one): it runs on a second stream after everything recorded before it, and the next
 * lrm_hip_barrier, or the end of the list, waits for it. For read-only side work such as cache prefetch. */
int lrm_hip_dispatch_overlapped(lrm_hip_list *l, uint32_t kernel, const uint32_t words[32]);
/* No counterpart in the reference. For callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops that forbid hipMalloc): records attention_decode_f16 followed by attention_combine (f32 output) with the
 * split partials in the library's static scratch, a 4 MiB array each GPU holds from the library's load until the
 * process ends, instead of a partials tensor of the caller's heap. words: the attention_decode_f16 argument block with
 * its partials word 0; y: the combine's output token, f32 [batch, q_heads * 128]. Raises LRM_E_CONTRACT when
 * batch * q_heads * splits * 130 * 4 bytes exceed the scratch. Records nothing that allocates; calls that overlap on one
 * GPU (lists from two backends of that GPU) share the scratch and race. */
int lrm_hip_dispatch_decode_attention_static(lrm_hip_list *l, const uint32_t words[32], uint32_t y);
/* ICommandList.Barrier: joins the overlapped dispatches (the in-order dispatches need nothing). */
int lrm_hip_barrier(lrm_hip_list *l);
int lrm_hip_copy(lrm_hip_list *l, int src_slot, uint64_t src_offset, int dst_slot, uint64_t dst_offset, uint64_t bytes);
int lrm_hip_begin_timer(lrm_hip_list *l, const char *name, int *timer);
int lrm_hip_end_timer(lrm_hip_list *l, int timer);
int lrm_hip_submit(lrm_hip_device *d, lrm_hip_list *l, uint32_t repeat, uint64_t *fence);
int lrm_hip_wait(lrm_hip_device *d, uint64_t fence, int *dispatches, int *timers);
int lrm_hip_timer(lrm_hip_device *d, uint64_t fence, int index, char *name, int name_cap, int64_t *start_ns,
                  int64_t *duration_ns);
int lrm_hip_release(lrm_hip_device *d, lrm_hip_list *l); /* frees a reusable list */

/* ======================================================================== the Qwen3 executor
 * The counterpart of the planned Lrm.Gpu.Exec GpuForwardOps and Lrm.Models.Qwen Forward/Greedy (docs/dev-plan.md:
 * 166-170,205-209,289-290), whose only existing form is tests/Lrm.Tensor.Tests/TinyModel.fs:144-236. mode 0 runs the
 * reference catalog kernels in fp32 (parity with CpuRef F32); mode 1 runs the fast path (bf16 weights; fp16 MFMA
 * operands and an fp16 KV cache in prefill; bf16-weight GEMVs for one sequence in decode). */
typedef struct lrm_qwen_config {
    int32_t layers, hidden, heads, kv_heads, head_dim, intermediate, vocab, max_pos;
    float eps;
    int32_t mode;       /* 0 fp32 catalog, 1 fast */
    int32_t max_tokens; /* rows per forward chunk */
    int32_t batch;      /* sequences with their own KV cache: 1 (mode 0), 1 .. 16 (mode 1) */
    int32_t taps;       /* mode 0: keep every ActivationNames tap (src/Lrm.Tensor/Goldens.fs:288-322) */
} lrm_qwen_config;

typedef struct lrm_qwen lrm_qwen;
/* inv_freq_bits: the pinned float32 inverse frequencies, head_dim / 2 words (Rope.fs:218-251). */
int lrm_qwen_create(lrm_hip_device *d, const lrm_qwen_config *cfg, const uint32_t *inv_freq_bits, int half,
                    lrm_qwen **out);
int lrm_qwen_destroy(lrm_qwen *q);
/* Weights by Hugging Face name, bf16 bits (TinyModel.fs:79-101 names; tied lm_head = model.embed_tokens.weight). */
int lrm_qwen_set_weight(lrm_qwen *q, const char *name, const uint16_t *data, uint64_t elems);
int lrm_qwen_read_weight(lrm_qwen *q, const char *name, uint16_t *out, uint64_t elems);
/* Every weight from a Qwen3 checkpoint (model.safetensors) through the validating reader below: each weight of the
 * configuration present as BF16 with its exact shape, no other tensor but an optional lm_head.weight that must equal
 * model.embed_tokens.weight byte for byte (Qwen3 ties them; the Qwen3-0.6B file stores both: 311 entries,
 * tests/Lrm.Tensor.Tests/ModelTests.fs:16-29). Uploads straight from the mapped file in pieces of at most 64 MiB
 * (UploadFrom, src/Lrm.Gpu.Core/Backend.fs:119-120). LRM_E_FORMAT for a malformed file, LRM_E_ARG for a file of
 * another layout. */
int lrm_qwen_load_safetensors(lrm_qwen *q, const char *path);
/* TinyModel.forward (TinyModel.fs:144-204): ids at positions pos0 .. pos0 + t - 1; writes the cache; the last
 * logits_rows rows of logits (f32 [logits_rows, vocab]) when logits != NULL; *argmax = argmax of the last row
 * (0xFFFFFFFF for a row holding a NaN, argmaxRows semantics). */
int lrm_qwen_forward(lrm_qwen *q, int seq, int pos0, const int32_t *ids, int t, float *logits, int logits_rows,
                     uint32_t *argmax);
/* TinyModel.greedy (TinyModel.fs:219-236): prefill then steps - 1 decode steps; mode 1 decodes on device. */
int lrm_qwen_greedy(lrm_qwen *q, const int32_t *prompt, int prompt_len, int steps, int32_t *out_ids);
/* On-device decode (mode 1): state = (token ids[b] at positions pos[b], one per sequence), run `steps` recorded decode
 * steps (one HIP graph replay each), read the ids they produced (out[s * batch + b] = the id sequence b chose at step
 * s). One sequence decodes with GEMVs over the bf16 weights; 2 .. 16 together with skinny MFMA GEMMs over the fp16
 * copies (config E of the hot path: the 1.7B shape, 16 sequences at 8K context). */
int lrm_qwen_decode_set(lrm_qwen *q, const int32_t *ids, const int32_t *pos);
int lrm_qwen_decode_run(lrm_qwen *q, int steps);
int lrm_qwen_decode_ids(lrm_qwen *q, int32_t *out, int count);
/* decode_set + decode_run(steps) + decode_ids(steps * batch): the batched greedy loop on device. */
int lrm_qwen_decode_batch(lrm_qwen *q, const int32_t *ids, const int32_t *pos, int steps, int32_t *out_ids);
/* Rows of the logits buffer: after a decode step, row 0 holds that step's logits. */
int lrm_qwen_read_logits(lrm_qwen *q, float *out, int rows);
double lrm_qwen_last_ms(lrm_qwen *q); /* device time of the last forward / decode run, ms */
/* 1 when the one-sequence decode step runs as the single persistent launch (catalog kernel decode_step_persistent:
 * all layers in one dispatch, stages handed over through tagged exchange entries), 0 when it runs as the recorded list
 * of per-stage kernels, -1 for a null model. No counterpart in the reference: its decode loop is the planned
 * Lrm.Gpu.Exec composition of per-op dispatches (docs/dev-plan.md:166-170), which the per-stage list mirrors. */
int lrm_qwen_persistent_decode(lrm_qwen *q);
/* Mode 1: the binades s by which the SwiGLU output is shifted down before it is stored as fp16 (a 2^-s; the down_proj
 * GEMM multiplies its sums by 2^s, so every result equals the unshifted one while a 2^-s stays a normal fp16 number).
 * 0 until a forward's SwiGLU output overflows fp16; that forward then runs again with s raised by 8, up to 16, and s
 * stays for later calls until a weight is written. A decode call that overflows there fails and raises s for the calls
 * after it. -1 for a null model. No counterpart in the reference, whose kernels keep these activations in float32. */
int lrm_qwen_swiglu_shift(lrm_qwen *q);
/* Sets s (0 .. 24) for the calls that follow, until a weight is written or an overflow raises it: for a checkpoint
 * whose SwiGLU range is known ahead, which then needs no rerun. LRM_E_ARG outside that range or in mode 0. */
int lrm_qwen_set_swiglu_shift(lrm_qwen *q, int shift);
int lrm_qwen_token(lrm_qwen *q, const char *name, uint32_t *token);
lrm_hip_device *lrm_qwen_device(lrm_qwen *q);
int lrm_qwen_tap_count(lrm_qwen *q);
int lrm_qwen_tap_info(lrm_qwen *q, int i, char *name, int name_cap, int *width);
int lrm_qwen_read_tap(lrm_qwen *q, int i, float *out, int rows);
/* KV cache rows (which: 0 = K after norm and RoPE, 1 = V) as f32 [rows, kv_heads * head_dim]. */
int lrm_qwen_read_cache(lrm_qwen *q, int seq, int layer, int which, int row0, int rows, float *out);
int lrm_qwen_write_cache(lrm_qwen *q, int seq, int layer, int which, int row0, int rows, const float *in);
int lrm_qwen_fill_cache_random(lrm_qwen *q, uint64_t seed, int rows);

/* ======================================================================== inputs
 * Synthetic N(0, std) values (counter-based, thread-count independent) and the T_spec RoPE table. */
uint64_t lrm_stream_of(const char *name);
int lrm_synth_normal_f32(uint64_t seed, uint64_t stream, uint64_t n, float std, float *out);
int lrm_synth_normal_bf16(uint64_t seed, uint64_t stream, uint64_t n, float std, uint16_t *out);
int lrm_rope_table(const uint32_t *inv_freq_bits, int half, int max_pos, float *cos_out, float *sin_out);

/* ---- safetensors: the validating reader (SafetensorsFile, src/Lrm.Tensor/Safetensors.fs:504-727) ----
 * Open maps the file read-only and checks the 8-byte header length (at most 100,000,000), that the header is UTF-8
 * JSON (nesting at most 8) whose keys are unique, that every entry has exactly dtype (F32, BF16, F16, I32, U32, U8,
 * F64, I64), shape (non-negative integers) and data_offsets (a pair) with a byte count that matches, that metadata is
 * an object of strings, and that the tensors tile the data section exactly (SafetensorsParse.header, :401-498).
 * Entries and metadata come back in code point order of their names. Names are UTF-8 and may hold any character, so
 * they are returned as (bytes, length), not NUL-terminated. */
typedef struct lrm_st lrm_st;
int lrm_st_open(const char *path, lrm_st **out);                                   /* SafetensorsFile.Open */
int lrm_st_open_verified(const char *path, int64_t bytes, const char *sha256_hex, lrm_st **out); /* .OpenVerified */
int lrm_st_validate(const uint8_t *bytes, uint64_t n, lrm_st **out);               /* SafetensorsFile.Validate */
/* HeaderLength, DataOffset, Entries.Length, Metadata.Length, IsAligned, Length */
int lrm_st_info(const lrm_st *f, int64_t *header_length, int64_t *data_offset, int32_t *entries, int32_t *metadata,
                int32_t *aligned, uint64_t *length);
/* Entry i: up to name_cap bytes of its name (*name_len = the full length), dtype code, rank and up to dims_cap dims,
 * data offsets [begin, end) from the start of the data section. */
int lrm_st_entry(const lrm_st *f, int i, char *name, int name_cap, int32_t *name_len, uint32_t *dtype, int32_t *rank,
                 int64_t *dims, int dims_cap, int64_t *begin, int64_t *end);
int lrm_st_metadata(const lrm_st *f, int i, char *key, int key_cap, int32_t *key_len, char *value, int value_cap,
                    int32_t *value_len);
/* A pointer to entry i's bytes in the mapping, valid until lrm_st_close (SafetensorsFile.Span); i = -1: the file's
 * first byte (HeaderBytes). */
int lrm_st_data(const lrm_st *f, int i, const void **data);
int lrm_st_close(lrm_st *f);

/* ---- tokenizer: the Qwen3 byte-level BPE tokenizer (QwenTokenizer, src/Lrm.Tokenizer/QwenTokenizer.fs) ----
 * Encode: added tokens on the raw text (leftmost-longest), then for each stretch between them the oracle's NFC, the
 * Split pre-tokenizer and byte-level BPE; no BOS or EOS. Output arrays follow one rule: when the buffer is NULL or
 * `cap` is smaller than the result, nothing is written; *count (*len) is the result's size either way. */
typedef struct lrm_tok lrm_tok;
/* QwenTokenizer.parse: tokenizer.json bytes with the loader's checks (TokenizerJson.parse, TokenizerJson.fs:227-250):
 * LRM_E_DATA for any configuration other than Qwen3's. */
int lrm_tok_parse(const uint8_t *json, uint64_t n, lrm_tok **out);
int lrm_tok_destroy(lrm_tok *t);
int lrm_tok_info(const lrm_tok *t, int32_t *vocab_size, int32_t *merges, int32_t *added); /* VocabSize, MergeCount */
int lrm_tok_added(const lrm_tok *t, int i, int32_t *id, char *content, int cap, int32_t *len, int32_t *special);
/* Encode (UTF-8 text; LRM_E_ARG for ill-formed UTF-8, the reference's refusal of a lone surrogate) and EncodeBytes
 * (each maximal ill-formed subpart becomes U+FFFD first). */
int lrm_tok_encode(const lrm_tok *t, const uint8_t *utf8, uint64_t n, int32_t *ids, uint64_t cap, uint64_t *count);
int lrm_tok_encode_bytes(const lrm_tok *t, const uint8_t *bytes, uint64_t n, int32_t *ids, uint64_t cap,
                         uint64_t *count);
/* DecodeBytes: LRM_E_ARG for an id outside [0, 151936); ids from VocabSize up to 151936 give no bytes. */
int lrm_tok_decode_bytes(const lrm_tok *t, const int32_t *ids, uint64_t n, uint8_t *out, uint64_t cap, uint64_t *len);
int lrm_tok_id_of(const lrm_tok *t, const uint8_t *token, uint64_t n, int32_t *id); /* IdOf; -1 for none */
int lrm_tok_token_of(const lrm_tok *t, int32_t id, char *out, int cap, int32_t *len); /* TokenOf; *len -1: none */
/* The stages alone, for their tests: PreTokenizer.split (piece start byte offsets, then the text's length), Nfc.normalize,
 * and per scalar 0 .. 0x10FFFF the Split class (0 letter, 1 number, 2 space, 3 other), the contraction letter (0 for
 * none) and whether NFC splits there (each array 0x110000 bytes, NULL to skip), and the byte map. */
int lrm_tok_pre_split(const uint8_t *utf8, uint64_t n, uint64_t *bounds, uint64_t cap, uint64_t *count);
int lrm_tok_nfc(const uint8_t *utf8, uint64_t n, uint8_t *out, uint64_t cap, uint64_t *len);
/* Nfc.normalize of many strings at once: string i is text[offsets[i] .. offsets[i + 1]) (count + 1 offsets); the
 * results are concatenated in out, string i at out_offsets[i] .. out_offsets[i + 1]. */
int lrm_tok_nfc_many(const uint8_t *text, const uint64_t *offsets, uint64_t count, uint8_t *out, uint64_t cap,
                     uint64_t *out_offsets, uint64_t *len);
int lrm_tok_scalar_tables(uint8_t *classes, uint8_t *contraction, uint8_t *nfc_split);
int lrm_tok_byte_char(int b, uint32_t *c);

#ifdef __cplusplus
}
#endif

#endif
