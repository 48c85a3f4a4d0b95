// The Qwen3 executor: the counterpart of the reference's planned Lrm.Gpu.Exec GpuForwardOps and Lrm.Models.Qwen
// forward/greedy (docs/dev-plan.md:166-170,205-209,289-290; the only composition that exists in the reference is
// tests/Lrm.Tensor.Tests/TinyModel.fs:144-236). It drives the HIP device only through the contract: a two-pass static
// plan (HeapPlanner, then TensorTable + seal), CreateHeap, WriteTable, Upload/Download, and command lists of catalog
// dispatches.
//
// Two modes:
//   Fp32 - the reference catalog kernels (ids 0..13): fp32 activations and an fp32 token-major KV cache, as every
//          reference GPU keeps. This is the parity path against CpuRef F32.
//   Fast - the appended kernels: bf16 weights, fp16 MFMA operands in prefill (an exact on-device fp16 copy of each
//          matrix, fp16-rounded activations), fp32 residual stream, a head-major fp16 KV cache, fused
//          norm/RoPE/KV-append/SwiGLU/residual epilogues, and the decode step recorded once as a reusable list (a
//          hipGraph) that streams the bf16 weights, reads its position from device memory and feeds the greedy argmax
//          back on device.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <vector>

#include "contract.hpp"
#include "device.hpp"

namespace lrm {

struct QwenConfig {
    int layers, hidden, heads, kv_heads, head_dim, intermediate, vocab, max_pos;
    float eps;
    int mode;        // 0 = Fp32, 1 = Fast
    int max_tokens;  // rows per forward (prefill chunk); decode uses 1 per sequence
    int batch;       // sequences decoded together (Fast mode); 1 otherwise
    int taps;        // Fp32 mode: keep every ActivationNames tap of the last forward
};

class QwenExec {
  public:
    QwenExec(Device& dev, const QwenConfig& cfg, const uint32_t* inv_freq_bits);
    ~QwenExec();

    // Weights by their Hugging Face names (bf16 bits).
    void set_weight(const std::string& name, const uint16_t* data, uint64_t elems);
    // Every weight from a Qwen3 checkpoint in safetensors form (the validating reader): each weight of this
    // configuration present as bf16 with its exact shape, nothing else but an optional lm_head.weight identical to
    // the tied embedding.
    void load_safetensors(const std::string& path);
    std::vector<std::string> weight_names() const;
    void read_weight(const std::string& name, uint16_t* out, uint64_t elems);

    // One forward over ids at positions pos0.. for sequence `seq` (TinyModel.forward). logits_rows of the last rows of
    // logits are downloaded into `logits` (nullable); returns the argmax of the last row (0xFFFFFFFF for a NaN row).
    uint32_t forward(int seq, int pos0, const int32_t* ids, int t, float* logits, int logits_rows);
    // The canonical greedy schedule (TinyModel.greedy): prefill, then steps - 1 decode steps.
    void greedy(const int32_t* prompt, int prompt_len, int steps, int32_t* out_ids);
    // Batched greedy decode in Fast mode: positions pos[b] hold the next token ids[b] for every sequence; runs
    // `steps` decode steps on device and writes out_ids[s * batch + b].
    void decode_batch(const int32_t* ids, const int32_t* pos, int steps, int32_t* out_ids);

    // Taps of the last forward (Fp32 mode with taps): ActivationNames order, [t, width] f32.
    int tap_count() const;
    std::string tap_name(int i) const;
    int tap_width(int i) const;
    void read_tap(int i, float* out, int rows);
    // Cache rows [row0, row0 + rows) of layer `layer` (k or v) for sequence seq, as f32 [rows, kv_heads * head_dim].
    void read_cache(int seq, int layer, int which, int row0, int rows, float* out);
    // Writes cache rows from f32 (narrowed to the cache dtype): for synthetic long-context workloads.
    void write_cache(int seq, int layer, int which, int row0, int rows, const float* in);
    // Fills every sequence's cache rows [0, rows) of every layer with N(0, 1) on device (bf16 caches only).
    void fill_cache_random(uint64_t seed, int rows);

    // Timing of the last forward/decode submission as measured by device events (ms).
    double last_ms() const { return last_ms_; }
    const QwenConfig& config() const { return cfg_; }
    Device& device() { return dev_; }
    uint32_t token(const std::string& name) const;
    void run_decode_steps(int steps);  // Fast mode: replays the recorded decode step `steps` times (state on device)
    void set_decode_state(const int32_t* ids, const int32_t* pos);
    void read_decode_ids(int32_t* out, int count);
    // Fast mode, one sequence: true when the decode step is the single persistent launch (decode_step_persistent),
    // false when it is the recorded list of per-stage kernels. The persistent step is used when the device has at least
    // 256 CUs, the kernel covers the shape and LRM_HIP_DECODE is not "kernels" at construction.
    bool persistent_decode() const { return persist_; }
    // Fast mode: the binades s by which the SwiGLU output a is shifted down before it is stored as fp16 (a 2^-s; the
    // down_proj GEMM multiplies its sums by 2^s). 0 until a forward overflows there, which then reruns with
    // s = 8, then 16; any weight write sets it back to 0.
    int swiglu_shift() const { return swiglu_shift_; }
    // Sets s (0 .. kSwigluShiftLimit, the largest a_shift the kernels take) ahead of the next call: for a checkpoint
    // whose SwiGLU range is known, which then needs no rerun.
    void set_swiglu_shift_checked(int s);
    static constexpr int kSwigluShiftLimit = 24;
    static constexpr int kSwigluShiftStep = 8;
    static constexpr int kMaxSwigluShift = 16;

  private:
    void plan();
    void upload_rope(const uint32_t* inv_freq_bits);
    uint32_t forward_fp32(int pos0, int t, float* logits, int logits_rows);
    uint32_t forward_fast(int seq, int pos0, int t, float* logits, int logits_rows);
    uint32_t forward_chunks(int seq, int pos0, const int32_t* ids, int t, float* logits, int logits_rows);
    void set_swiglu_shift(int s);
    void set_weight_bytes(const std::string& name, const uint8_t* data, uint64_t elems);
    // Fast mode: fails the call (RangeError) naming the fp16 range sites in bits.
    [[noreturn]] void throw_f16_range(const char* what, uint32_t bits);
    void record_decode_fast();
    void record_decode_batch(CommandList* l);
    void sync_f16();  // refreshes the fp16 copies of the matrices written since the last forward
    void tap_copy(CommandList* l, const std::string& name, uint32_t src, int t, int width);
    uint32_t dispatch(CommandList* l, const char* kernel, std::vector<uint32_t> fields, bool overlapped = false);

    Device& dev_;
    QwenConfig cfg_;
    HeapPlanner planner_;
    std::unique_ptr<TensorTable> table_;
    struct Tensor {
        Placement place;
        uint32_t dtype;
        std::vector<uint32_t> dims;
        uint32_t flags;
        uint32_t token = 0;
        std::string view_of;  // non-empty: a view of another tensor
        uint64_t view_offset = 0;
    };
    std::map<std::string, Tensor> tensors_;
    std::vector<std::string> order_;
    std::vector<std::string> weight_names_;
    std::vector<std::string> tap_names_;
    std::vector<int> tap_widths_;
    int last_t_ = 0;
    double last_ms_ = 0;
    CommandList* decode_list_ = nullptr;
    bool persist_ = false;    // the decode step is decode_step_persistent (layer-stacked weights and caches)
    int persist_blocks_ = 0;  // its workgroups
    int swiglu_shift_ = 0;
    std::map<std::string, std::string> f16_copy_;  // bf16 matrix -> its fp16 copy (Fast mode)
    std::set<std::string> f16_dirty_;
    void add(const std::string& name, uint32_t arena, uint32_t dtype, std::vector<uint32_t> dims, uint32_t flags = 0);
    void add_view(const std::string& name, const std::string& of, std::vector<uint32_t> dims, uint64_t elem_offset);
    const Tensor& t(const std::string& name) const;
    void upload_tensor(const std::string& name, const void* data, uint64_t bytes, uint64_t byte_offset = 0);
    void download_tensor(const std::string& name, void* out, uint64_t bytes, uint64_t byte_offset = 0);
};

// Host synthetic inputs: a counter-based normal generator (splitmix64 of (seed, stream, index), Box-Muller), so every
// element is a pure function of its coordinates and the bits do not depend on the thread count.
void synth_normal_f32(uint64_t seed, uint64_t stream, uint64_t n, float std, float* out);
void synth_normal_bf16(uint64_t seed, uint64_t stream, uint64_t n, float std, uint16_t* out);
uint64_t stream_of(const char* name);  // FNV-1a 64 of a tensor name

// The T_spec RoPE table of the product (Rope.fs:218-251): freq = f32(f32(pos) * inv_freq[j]), cos/sin =
// f32(RN64(cos/sin freq)) with a certified binary128 evaluation. Throws when a rounding cannot be certified.
void rope_table(const uint32_t* inv_freq_bits, int half, int max_pos, float* cos_out, float* sin_out);

}  // namespace lrm
