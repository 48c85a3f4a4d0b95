// The Qwen3 executor (see qwen_exec.hpp).
#include "qwen_exec.hpp"
#include "safetensors.hpp"

#include "attn_prefill.hpp"
#include "kv_layout.hpp"
#include "persist.hpp"

#include <omp.h>
#include <quadmath.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdlib>
#include <cstring>

namespace lrm {

static uint32_t fbits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

static void arg_fail(const char* fmt, ...) __attribute__((format(printf, 1, 2), noreturn));
static void arg_fail(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    throw std::invalid_argument(buf);
}

// ---------------------------------------------------------------- T_spec (Rope.fs:146-161, 218-251)
// The correctly rounded float64 cos/sin of a float32: binary128 evaluation, accepted only when the value is farther
// than 2^-100 (relative) from a float64 rounding boundary, so a binary128 error of a few ulps cannot cross it.
static bool round_certain(__float128 v, double* out) {
    double d = double(v);
    if (v == __float128(d)) {
        *out = d;
        return true;
    }
    __float128 lo = (__float128(d) + __float128(std::nextafter(d, -INFINITY))) / 2;
    __float128 hi = (__float128(d) + __float128(std::nextafter(d, INFINITY))) / 2;
    __float128 tol = fabsq(v) * __float128(0x1p-100);
    if (v - lo > tol && hi - v > tol) {
        *out = d;
        return true;
    }
    return false;
}

void rope_table(const uint32_t* inv, int half, int max_pos, float* cos_out, float* sin_out) {
    if (half < 1 || max_pos < 1 || max_pos > (1 << 24)) arg_fail("rope table: half %d, max_pos %d", half, max_pos);
    int bad = 0;
#pragma omp parallel for schedule(dynamic, 16)
    for (int pos = 0; pos < max_pos; ++pos) {
        for (int j = 0; j < half; ++j) {
            float f;
            std::memcpy(&f, &inv[j], 4);
            volatile float fp = float(pos);
            float x = fp * f;
            double c, s;
            if (!std::isfinite(x)) {
                c = s = NAN;
            } else if (std::fabs(x) < 0x1p-27f) {
                c = 1.0;
                s = double(x);
            } else {
                __float128 sq, cq;
                sincosq(__float128(std::fabs(x)), &sq, &cq);
                if (!round_certain(cq, &c) || !round_certain(sq, &s)) {
#pragma omp atomic write
                    bad = 1;
                }
                if (x < 0) s = -s;
            }
            cos_out[size_t(pos) * half + j] = float(c);
            sin_out[size_t(pos) * half + j] = float(s);
        }
    }
    if (bad) throw std::runtime_error("rope table: a cos/sin rounding could not be certified");
}

// ---------------------------------------------------------------- synthetic inputs

static uint64_t splitmix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t stream_of(const char* name) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (const char* p = name; *p; ++p) h = (h ^ uint8_t(*p)) * 0x100000001b3ull;
    return h;
}

void synth_normal_f32(uint64_t seed, uint64_t stream, uint64_t n, float std_, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t pi = 0; pi < int64_t((n + 1) / 2); ++pi) {
        uint64_t i = uint64_t(pi) * 2;
        uint64_t h = splitmix(seed ^ splitmix(stream ^ splitmix(i >> 1)));
        double u1 = (double((h >> 11) & ((1ull << 26) - 1)) + 0.5) / double(1ull << 26);
        double u2 = double(h >> 38) / double(1ull << 26);
        double r = std::sqrt(-2.0 * std::log(u1));
        out[i] = float(std_ * r * std::cos(6.283185307179586 * u2));
        if (i + 1 < n) out[i + 1] = float(std_ * r * std::sin(6.283185307179586 * u2));
    }
}

static uint16_t narrow_rne(float f) {
    uint32_t u = fbits(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u & 0x80000000u) ? 0xFFC0 : 0x7FC0;
    return uint16_t((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

void synth_normal_bf16(uint64_t seed, uint64_t stream, uint64_t n, float std_, uint16_t* out) {
#pragma omp parallel for schedule(static)
    for (int64_t pi = 0; pi < int64_t((n + 1) / 2); ++pi) {
        uint64_t i = uint64_t(pi) * 2;
        uint64_t h = splitmix(seed ^ splitmix(stream ^ splitmix(i >> 1)));
        double u1 = (double((h >> 11) & ((1ull << 26) - 1)) + 0.5) / double(1ull << 26);
        double u2 = double(h >> 38) / double(1ull << 26);
        double r = std::sqrt(-2.0 * std::log(u1));
        out[i] = narrow_rne(float(std_ * r * std::cos(6.283185307179586 * u2)));
        if (i + 1 < n) out[i + 1] = narrow_rne(float(std_ * r * std::sin(6.283185307179586 * u2)));
    }
}

// ---------------------------------------------------------------- plan

static const char* kLayerWeights[11] = {"input_layernorm.weight", "self_attn.q_proj.weight", "self_attn.k_proj.weight",
                                        "self_attn.v_proj.weight", "self_attn.o_proj.weight", "self_attn.q_norm.weight",
                                        "self_attn.k_norm.weight", "post_attention_layernorm.weight",
                                        "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight"};

static const char* kLayerTaps[18] = {"input_layernorm.out", "attn.q_proj.out", "attn.k_proj.out", "attn.v_proj.out",
                                     "attn.q_norm.out", "attn.k_norm.out", "attn.q_rope", "attn.k_rope",
                                     "attn.v_cache", "attn.o_proj.in", "attn.o_proj.out", "resid_mid",
                                     "post_attention_layernorm.out", "mlp.gate.out", "mlp.up.out", "mlp.down.in",
                                     "mlp.down.out", "out"};

static std::string lname(int i, const char* n) { return "model.layers." + std::to_string(i) + "." + n; }

void QwenExec::add(const std::string& name, uint32_t arena, uint32_t dtype, std::vector<uint32_t> dims, uint32_t flags) {
    uint64_t elems = 1;
    for (uint32_t d : dims) elems *= d;
    uint64_t bytes = (elems * uint64_t(dtype_size(dtype)) + 3) / 4 * 4;
    Tensor t{};
    t.place = planner_.allocate(arena, bytes);
    t.dtype = dtype;
    t.dims = std::move(dims);
    t.flags = flags;
    tensors_[name] = t;
    order_.push_back(name);
}

void QwenExec::add_view(const std::string& name, const std::string& of, std::vector<uint32_t> dims, uint64_t elem_offset) {
    Tensor t{};
    t.dims = std::move(dims);
    t.view_of = of;
    t.view_offset = elem_offset;
    t.dtype = tensors_.at(of).dtype;
    tensors_[name] = t;
    order_.push_back(name);
}

const QwenExec::Tensor& QwenExec::t(const std::string& name) const {
    auto it = tensors_.find(name);
    if (it == tensors_.end()) arg_fail("no tensor '%s' in the plan", name.c_str());
    return it->second;
}

uint32_t QwenExec::token(const std::string& name) const { return t(name).token; }

QwenExec::QwenExec(Device& dev, const QwenConfig& cfg, const uint32_t* inv_freq_bits) : dev_(dev), cfg_(cfg) {
    const QwenConfig& c = cfg_;
    if (c.layers < 1 || c.hidden < 1 || c.heads < 1 || c.kv_heads < 1 || c.head_dim < 2 || c.intermediate < 1 ||
        c.vocab < 1 || c.max_pos < 1 || c.max_tokens < 1)
        arg_fail("a Qwen3 config needs positive sizes");
    if (c.heads % c.kv_heads) arg_fail("kv_heads must divide heads");
    if (c.head_dim % 2) arg_fail("head_dim must be even");
    if (c.mode == 1) {
        if (c.head_dim != 128 || c.heads != 2 * c.kv_heads)
            arg_fail("the fast path takes head_dim 128 and two query heads per KV head");
        if (c.hidden % 64 || c.intermediate % 64 || c.hidden > 8192 || c.intermediate > 8192 || c.heads * 128 > 8192)
            arg_fail("the fast path takes hidden and intermediate multiples of 64 up to 8192, and heads * 128 <= 8192");
        if (c.max_pos % 64 || c.max_pos > 65536) arg_fail("the fast path takes max_pos a multiple of 64 up to 65536");
        if (c.batch < 1 || c.batch > 16) arg_fail("the fast path decodes 1 .. 16 sequences together");
        if (c.batch > 1 && (c.hidden % 1024 || c.intermediate % 1024 || (c.heads * 128) % 1024 || c.max_tokens < c.batch))
            arg_fail("batched decode takes hidden, intermediate and heads * 128 multiples of 1024, and max_tokens >= batch");
    } else if (c.batch != 1) {
        arg_fail("the fp32 mode holds one sequence");
    }
    // each mode runs under its kernel set's ExecutionClass: fp32 the reference set, fast the fast set (a fast-set
    // device also runs the fp32 mode, whose results it then classes as the fast set's)
    const Device::KernelSet need = c.mode == 0 ? Device::KernelSet::Reference : Device::KernelSet::Fast;
    if (!dev_.kernels_loaded()) dev_.load_kernels(need);
    if (c.mode != 0 && dev_.kernel_set() != Device::KernelSet::Fast)
        arg_fail("the fast mode needs a device with the fast kernel set loaded (lrm_hip_load_kernel_set, "
                 "LRM_HIP_KERNELS_FAST); this one has the reference set");
    plan();
    upload_rope(inv_freq_bits);
}

QwenExec::~QwenExec() {
    if (decode_list_) dev_.release(decode_list_);
}

void QwenExec::plan() {
    const QwenConfig& c = cfg_;
    const uint32_t H = c.hidden, QC = c.heads * c.head_dim, KC = c.kv_heads * c.head_dim, I = c.intermediate,
                   V = c.vocab, MT = c.max_tokens, MP = c.max_pos, HD = c.head_dim;
    const bool fast = c.mode == 1;
    const uint32_t L = uint32_t(c.layers), KVH = uint32_t(c.kv_heads), N1 = QC + 2 * KC;
    // The one-launch decode step (one sequence) reads every layer through layer-stacked tensors, one per kind; the
    // per-layer names are views of them. Each stack must fit one heap page.
    if (fast && c.batch == 1) {
        const char* env = std::getenv("LRM_HIP_DECODE");
        const bool want = !(env && std::string(env) == "kernels");
        const int G = 256;
        const persist::Shape sh{c.hidden, c.heads, c.kv_heads, c.head_dim, c.intermediate, c.max_pos, G};
        auto fits = [](uint64_t elems) { return elems * 2 <= kMaxPageBytes; };
        persist_ = want && dev_.info().compute_units >= G && !persist::unsupported(sh) && fits(uint64_t(L) * N1 * H) &&
                   fits(uint64_t(L) * 2 * I * H) && fits(uint64_t(L) * H * QC) && fits(uint64_t(L) * H * I) &&
                   fits(uint64_t(L) * KVH * MP * HD);
        persist_blocks_ = G;
    }
    // pass one: placements (HeapLayout.fs:433-525); weights first, in contract arena order
    add("model.embed_tokens.weight", Weights, BF16, {V, H}, ReadOnly);
    add("model.norm.weight", Weights, BF16, {H}, ReadOnly);
    if (persist_) {
        add("stack.input_layernorm", Weights, BF16, {L, H}, ReadOnly);
        add("stack.qkv_proj", Weights, BF16, {L, N1, H}, ReadOnly);
        add("stack.o_proj", Weights, BF16, {L, H, QC}, ReadOnly);
        add("stack.q_norm", Weights, BF16, {L, HD}, ReadOnly);
        add("stack.k_norm", Weights, BF16, {L, HD}, ReadOnly);
        add("stack.post_attention_layernorm", Weights, BF16, {L, H}, ReadOnly);
        add("stack.gate_up_proj", Weights, BF16, {L, 2 * I, H}, ReadOnly);
        add("stack.down_proj", Weights, BF16, {L, H, I}, ReadOnly);
        for (uint32_t i = 0; i < L; ++i) {
            add_view(lname(int(i), kLayerWeights[0]), "stack.input_layernorm", {H}, uint64_t(i) * H);
            add_view("L" + std::to_string(i) + ".qkv_proj", "stack.qkv_proj", {N1, H}, uint64_t(i) * N1 * H);
            add_view(lname(int(i), kLayerWeights[4]), "stack.o_proj", {H, QC}, uint64_t(i) * H * QC);
            add_view(lname(int(i), kLayerWeights[5]), "stack.q_norm", {HD}, uint64_t(i) * HD);
            add_view(lname(int(i), kLayerWeights[6]), "stack.k_norm", {HD}, uint64_t(i) * HD);
            add_view(lname(int(i), kLayerWeights[7]), "stack.post_attention_layernorm", {H}, uint64_t(i) * H);
            add_view("L" + std::to_string(i) + ".gate_up_proj", "stack.gate_up_proj", {2 * I, H}, uint64_t(i) * 2 * I * H);
            add_view(lname(int(i), kLayerWeights[10]), "stack.down_proj", {H, I}, uint64_t(i) * H * I);
        }
    }
    for (int i = 0; i < c.layers && !persist_; ++i) {
        add(lname(i, kLayerWeights[0]), Weights, BF16, {H}, ReadOnly);
        if (fast) {
            add("L" + std::to_string(i) + ".qkv_proj", Weights, BF16, {QC + 2 * KC, H}, ReadOnly);
        } else {
            add(lname(i, kLayerWeights[1]), Weights, BF16, {QC, H}, ReadOnly);
            add(lname(i, kLayerWeights[2]), Weights, BF16, {KC, H}, ReadOnly);
            add(lname(i, kLayerWeights[3]), Weights, BF16, {KC, H}, ReadOnly);
        }
        add(lname(i, kLayerWeights[4]), Weights, BF16, {H, QC}, ReadOnly);
        add(lname(i, kLayerWeights[5]), Weights, BF16, {HD}, ReadOnly);
        add(lname(i, kLayerWeights[6]), Weights, BF16, {HD}, ReadOnly);
        add(lname(i, kLayerWeights[7]), Weights, BF16, {H}, ReadOnly);
        if (fast) {
            add("L" + std::to_string(i) + ".gate_up_proj", Weights, BF16, {2 * I, H}, ReadOnly);
        } else {
            add(lname(i, kLayerWeights[8]), Weights, BF16, {I, H}, ReadOnly);
            add(lname(i, kLayerWeights[9]), Weights, BF16, {I, H}, ReadOnly);
        }
        add(lname(i, kLayerWeights[10]), Weights, BF16, {H, I}, ReadOnly);
    }
    if (fast) {
        // exact fp16 copies of the matrices for the prefill MFMA GEMMs (and the persistent decode step), written on
        // device from the bf16 originals; layer-stacked like the originals when the decode step is persistent
        auto copy16 = [&](const std::string& of, const std::string& name, std::vector<uint32_t> dims) {
            add(name, Weights, F16, std::move(dims));
            f16_copy_[of] = name;
        };
        copy16("model.embed_tokens.weight", "embed.f16", {V, H});
        if (persist_) {
            add("stack.qkv_proj.f16", Weights, F16, {L, N1, H});
            add("stack.o_proj.f16", Weights, F16, {L, H, QC});
            add("stack.gate_up_proj.f16", Weights, F16, {L, 2 * I, H});
            add("stack.down_proj.f16", Weights, F16, {L, H, I});
        }
        auto view16 = [&](const std::string& of, const std::string& name, const std::string& stack,
                          std::vector<uint32_t> dims, uint64_t off) {
            if (!persist_) return copy16(of, name, std::move(dims));
            add_view(name, stack, std::move(dims), off);
            f16_copy_[of] = name;
        };
        for (int i = 0; i < c.layers; ++i) {
            std::string p = "L" + std::to_string(i);
            const uint64_t ui = uint64_t(i);
            view16(p + ".qkv_proj", p + ".qkv_proj.f16", "stack.qkv_proj.f16", {QC + 2 * KC, H}, ui * N1 * H);
            view16(lname(i, kLayerWeights[4]), p + ".o_proj.f16", "stack.o_proj.f16", {H, QC}, ui * H * QC);
            view16(p + ".gate_up_proj", p + ".gate_up_proj.f16", "stack.gate_up_proj.f16", {2 * I, H}, ui * 2 * I * H);
            view16(lname(i, kLayerWeights[10]), p + ".down_proj.f16", "stack.down_proj.f16", {H, I}, ui * H * I);
        }
    }
    add("rope.cos", Rope, F32, {MP, HD / 2}, ReadOnly);
    add("rope.sin", Rope, F32, {MP, HD / 2}, ReadOnly);
    if (persist_) {
        add("stack.k_cache", KvCache, F16, {L, KVH, MP, HD});
        add("stack.v_cache", KvCache, F16, {L, KVH, HD, MP});
    }
    for (int i = 0; i < c.layers; ++i) {
        std::string p = "L" + std::to_string(i);
        if (persist_) {
            add_view(p + ".k_cache", "stack.k_cache", {KVH, MP, HD}, uint64_t(i) * KVH * MP * HD);
            add_view(p + ".v_cache", "stack.v_cache", {KVH, HD, MP}, uint64_t(i) * KVH * MP * HD);
        } else if (fast) {  // sequence b's heads follow sequence b - 1's
            add(p + ".k_cache", KvCache, F16, {uint32_t(c.batch * c.kv_heads), MP, HD});
            add(p + ".v_cache", KvCache, F16, {uint32_t(c.batch * c.kv_heads), HD, MP});
        } else {
            add(p + ".k_cache", KvCache, F32, {MP, KC});
            add(p + ".v_cache", KvCache, F32, {MP, KC});
        }
    }
    add("ids", Activations, U32, {MT});
    add("x", Activations, F32, {MT, H});
    const uint32_t LC = std::min<uint32_t>(MT, 512);  // logits rows per lm_head dispatch (K2-0001's row cap, raised)
    if (fast) {
        add("h", Activations, F16, {MT, H});
        add("q", Activations, F16, {MT, QC});
        add("o", Activations, F16, {MT, QC});
        add("a", Activations, F16, {MT, I});
        add("resid.partials", Scratch, F32, {2 * MT, H});  // the k-split partials of the prefill residual GEMMs
        // the prefill attention's split-tile partials and counters (zeroed below; every launch leaves them zero)
        add("attn.ws", Scratch, U32, {uint32_t(attn_prefill::workspace_words(MT, KVH))});
        const uint32_t B = uint32_t(c.batch);
        add("dec.x", Activations, F32, {B, H});
        add("dec.qkv", Scratch, F32, {B, QC + 2 * KC});
        add("dec.attn_partials", Scratch, F32, {B * uint32_t(c.heads) * (MP / 64) * 130});
        add("dec.state", Scratch, U32, {2 * B + 2});  // pos[B], id[B], step
        add("argmax.partials", Scratch, F32, {std::min<uint32_t>(MT, 512) * 64 * 2});
        add("dec.out_ids", Logits, U32, {MP * B});
        if (B == 1) {  // GEMVs on the bf16 weights, f32 vectors
            add("dec.o", Activations, F32, {QC});
            add("dec.a", Activations, F32, {I});
            add("dec.lm_partials", Scratch, F32, {2 * 1024});
            if (persist_) {
                const persist::Shape sh{c.hidden, c.heads, c.kv_heads, c.head_dim, c.intermediate, c.max_pos,
                                        persist_blocks_};
                add("dec.exchange", Scratch, U32, {uint32_t(2 * persist::exchange_entries(c.layers, sh))});
            }
        } else {  // skinny MFMA GEMMs on the fp16 copies
            add("dec.h16", Activations, F16, {B, H});
            add("dec.o16", Activations, F16, {B, QC});
            add("dec.a16", Activations, F16, {B, I});
        }
    } else {
        for (const char* n : {"h", "oo", "r", "h2", "dd", "f"}) add(n, Activations, F32, {MT, H});
        for (const char* n : {"q", "qn", "qr", "o"}) add(n, Activations, F32, {MT, QC});
        for (const char* n : {"k", "v", "kn", "kr"}) add(n, Activations, F32, {MT, KC});
        for (const char* n : {"g", "u", "d"}) add(n, Activations, F32, {MT, I});
        add("f_last", Activations, F32, {LC, H});
    }
    add("logits", Logits, F32, {LC, V});
    add("argmax", Logits, U32, {LC});
    if (!fast && c.taps) {
        auto tap = [&](const std::string& n, uint32_t wdt) {
            add("tap." + n, Taps, F32, {MT, wdt});
            tap_names_.push_back(n);
            tap_widths_.push_back(int(wdt));
        };
        tap("embed.out", H);
        for (int i = 0; i < c.layers; ++i) {
            std::string p = "L" + std::to_string(i) + ".";
            uint32_t w[18] = {H, QC, KC, KC, QC, KC, QC, KC, KC, QC, H, H, H, I, I, I, H, H};
            for (int k = 0; k < 18; ++k) tap(p + kLayerTaps[k], w[k]);
        }
        tap("final_norm.out", H);
        tap("logits", V);
    }
    if (fast) {
        for (int i = 0; i < c.layers; ++i) {
            std::string p = "L" + std::to_string(i);
            add_view(lname(i, kLayerWeights[1]), p + ".qkv_proj", {QC, H}, 0);
            add_view(lname(i, kLayerWeights[2]), p + ".qkv_proj", {KC, H}, uint64_t(QC) * H);
            add_view(lname(i, kLayerWeights[3]), p + ".qkv_proj", {KC, H}, uint64_t(QC + KC) * H);
            for (int b = 0; b < c.batch; ++b) {
                const uint64_t off = uint64_t(b) * c.kv_heads * MP * HD;
                add_view(p + ".k_cache.s" + std::to_string(b), p + ".k_cache", {uint32_t(c.kv_heads), MP, HD}, off);
                add_view(p + ".v_cache.s" + std::to_string(b), p + ".v_cache", {uint32_t(c.kv_heads), HD, MP}, off);
            }
            add_view(lname(i, kLayerWeights[8]), p + ".gate_up_proj", {I, H}, 0);
            add_view(lname(i, kLayerWeights[9]), p + ".gate_up_proj", {I, H}, uint64_t(I) * H);
        }
    }
    // pass two: the layout, the table, the heap
    HeapLayout layout = planner_.build();
    table_.reset(new TensorTable(layout));
    for (const std::string& n : order_) {
        Tensor& tt = tensors_[n];
        if (tt.view_of.empty())
            tt.token = table_->add_placed(n, planner_, tt.place, tt.dtype, tt.dims, tt.flags);
        else
            tt.token = table_->add_view(n, tensors_[tt.view_of].token, tt.dims, tt.view_offset);
    }
    table_->seal();
    dev_.create_heap(layout);
    dev_.write_table(table_->image().data(), kTableBytes);
    if (persist_) {  // epoch 0, no abort, every entry untagged
        std::vector<uint8_t> zero(dev_.table().row(token("dec.exchange")).extent_bytes(), 0);
        upload_tensor("dec.exchange", zero.data(), zero.size());
    }
    if (fast) {
        std::vector<uint8_t> zero(dev_.table().row(token("attn.ws")).extent_bytes(), 0);
        upload_tensor("attn.ws", zero.data(), zero.size());
    }
    for (int i = 0; i < c.layers; ++i)
        for (int k = 0; k < 11; ++k) weight_names_.push_back(lname(i, kLayerWeights[k]));
    weight_names_.push_back("model.embed_tokens.weight");
    weight_names_.push_back("model.norm.weight");
}

void QwenExec::upload_tensor(const std::string& name, const void* data, uint64_t bytes, uint64_t byte_offset) {
    TensorRow r = dev_.table().row(token(name));
    if (byte_offset + bytes > r.extent_bytes()) arg_fail("%s holds %llu bytes", name.c_str(), (unsigned long long)r.extent_bytes());
    dev_.upload(int(r.slot()), r.offset() + byte_offset, data, bytes);
}

void QwenExec::download_tensor(const std::string& name, void* out, uint64_t bytes, uint64_t byte_offset) {
    TensorRow r = dev_.table().row(token(name));
    if (byte_offset + bytes > r.extent_bytes()) arg_fail("%s holds %llu bytes", name.c_str(), (unsigned long long)r.extent_bytes());
    dev_.download(int(r.slot()), r.offset() + byte_offset, out, bytes);
}

void QwenExec::upload_rope(const uint32_t* inv) {
    const int half = cfg_.head_dim / 2, mp = cfg_.max_pos;
    std::vector<float> cs(size_t(mp) * half), sn(size_t(mp) * half);
    rope_table(inv, half, mp, cs.data(), sn.data());
    upload_tensor("rope.cos", cs.data(), cs.size() * 4);
    upload_tensor("rope.sin", sn.data(), sn.size() * 4);
}

std::vector<std::string> QwenExec::weight_names() const { return weight_names_; }

void QwenExec::set_weight(const std::string& name, const uint16_t* data, uint64_t elems) {
    set_weight_bytes(name, reinterpret_cast<const uint8_t*>(data), elems);
}

// The bf16 elements as little-endian byte pairs (a mapped file need not align them), uploaded in pieces of at most
// 64 MiB.
void QwenExec::set_weight_bytes(const std::string& name, const uint8_t* data, uint64_t elems) {
    const Tensor& tt = t(name);
    uint64_t n = 1;
    for (uint32_t d : tt.dims) n *= d;
    if (tt.dtype != BF16 || n != elems) arg_fail("weight %s holds %llu bf16 elements, not %llu", name.c_str(), (unsigned long long)n, (unsigned long long)elems);
    const std::string base = f16_copy_.count(name) ? name : tt.view_of;  // the tensor with the fp16 copy, if any
    set_swiglu_shift(0);  // new weights: the next forward finds the shift they need
    if (f16_copy_.count(base)) {
        // the fp16 copy must hold the same values: |w| >= 65536 has no fp16 counterpart
        for (uint64_t i = 0; i < elems; ++i) {
            const uint16_t w = uint16_t(data[2 * i] | (uint16_t(data[2 * i + 1]) << 8)), a = w & 0x7FFFu;
            if (a >= 0x4780u && a < 0x7F80u)
                arg_fail("weight %s element %llu (bf16 %04x) is outside the fp16 range the fast path computes in",
                         name.c_str(), (unsigned long long)i, w);
        }
        f16_dirty_.insert(base);
    }
    constexpr uint64_t kPiece = uint64_t(64) << 20;
    for (uint64_t off = 0; off < elems * 2; off += kPiece)
        upload_tensor(name, data + off, std::min(kPiece, elems * 2 - off), off);
}

void QwenExec::load_safetensors(const std::string& path) {
    std::unique_ptr<StFile> f = StFile::open(path);
    const char* p = f->path().c_str();
    const std::set<std::string> expected(weight_names_.begin(), weight_names_.end());
    for (const StEntry& e : f->entries())
        if (e.name != "lm_head.weight" && !expected.count(e.name))
            arg_fail("%s: tensor %s is not a weight of this Qwen3 configuration", p, e.name.c_str());
    auto check = [&](const StEntry* e, const std::string& name, const std::vector<uint32_t>& dims) {
        if (!e) arg_fail("%s: no tensor %s", p, name.c_str());
        if (e->dtype != BF16) arg_fail("%s: %s is %s, not bf16", p, name.c_str(), dtype_name(e->dtype));
        bool same = e->shape.size() == dims.size();
        for (size_t k = 0; same && k < dims.size(); ++k) same = e->shape[k] == int64_t(dims[k]);
        if (!same) {
            std::string got, want;
            for (int64_t d : e->shape) got += (got.empty() ? "" : ", ") + std::to_string(d);
            for (uint32_t d : dims) want += (want.empty() ? "" : ", ") + std::to_string(d);
            arg_fail("%s: %s has shape [%s], not [%s]", p, name.c_str(), got.c_str(), want.c_str());
        }
    };
    for (const std::string& n : weight_names_) check(f->find(n), n, t(n).dims);
    // Qwen3 ties the output projection to the embedding: a stored lm_head must be a byte-exact copy of it
    const StEntry* emb = f->find("model.embed_tokens.weight");
    if (const StEntry* lm = f->find("lm_head.weight")) {
        check(lm, "lm_head.weight", t("model.embed_tokens.weight").dims);
        if (std::memcmp(f->data(*lm), f->data(*emb), size_t(emb->bytes())) != 0)
            arg_fail("%s: lm_head.weight differs from model.embed_tokens.weight; this executor ties them", p);
    }
    for (const std::string& n : weight_names_) {
        const StEntry* e = f->find(n);
        set_weight_bytes(n, f->data(*e), uint64_t(e->bytes() / 2));
    }
}

void QwenExec::sync_f16() {
    if (f16_dirty_.empty()) return;
    CommandList* l = dev_.begin();
    for (const std::string& base : f16_dirty_) {
        uint32_t n = dev_.table().row(token(base)).count();
        dispatch(l, "convert_bf16_f16", {token(base), token(f16_copy_.at(base)), n});
    }
    dev_.wait(dev_.submit(l));
    dev_.release(l);
    f16_dirty_.clear();
}

void QwenExec::read_weight(const std::string& name, uint16_t* out, uint64_t elems) {
    const Tensor& tt = t(name);
    uint64_t n = 1;
    for (uint32_t d : tt.dims) n *= d;
    if (n != elems) arg_fail("weight %s holds %llu elements", name.c_str(), (unsigned long long)n);
    download_tensor(name, out, elems * 2);
}

uint32_t QwenExec::dispatch(CommandList* l, const char* kernel, std::vector<uint32_t> fields, bool overlapped) {
    int id = catalog_find(kernel);
    if (id < 0) arg_fail("no kernel %s", kernel);
    uint32_t words[32] = {0};
    if (fields.size() > 31) arg_fail("too many fields");
    for (size_t i = 0; i < fields.size(); ++i) words[i + 1] = fields[i];
    if (overlapped)
        l->dispatch_overlapped(id, words);
    else
        l->dispatch(id, words);
    return uint32_t(id);
}

void QwenExec::tap_copy(CommandList* l, const std::string& name, uint32_t src, int rows, int width) {
    if (!cfg_.taps || cfg_.mode != 0) return;
    TensorRow s = dev_.table().row(src), d = dev_.table().row(token("tap." + name));
    l->copy(int(s.slot()), s.offset(), int(d.slot()), d.offset(), uint64_t(rows) * width * 4);
}

// ---------------------------------------------------------------- forward

uint32_t QwenExec::forward(int seq, int pos0, const int32_t* ids, int t_, float* logits, int logits_rows) {
    const QwenConfig& c = cfg_;
    if (seq < 0 || seq >= c.batch) arg_fail("sequence %d: %d planned", seq, c.batch);
    if (t_ < 1 || pos0 < 0 || pos0 + t_ > c.max_pos)
        arg_fail("positions %d .. %d outside max_pos %d", pos0, pos0 + t_ - 1, c.max_pos);
    if (logits_rows < 0 || logits_rows > t_) arg_fail("logits_rows %d outside 0 .. %d", logits_rows, t_);
    uint32_t am = 0xFFFFFFFFu;
    // Fast mode: a forward whose SwiGLU output left the fp16 range runs again with that output shifted down
    // kSwigluShiftStep binades more (the overflow may have spread to the sites after it, so those bits are no verdict
    // yet), up to kMaxSwigluShift; the shift then stays for later calls until a weight changes. Every rerun rewrites the
    // same cache rows and logits.
    for (;;) {
        am = forward_chunks(seq, pos0, ids, t_, logits, logits_rows);
        if (c.mode != 1) break;
        const uint32_t bits = dev_.take_f16_range();
        if ((bits & kF16SiteSwiglu) && swiglu_shift_ < kMaxSwigluShift) {
            set_swiglu_shift(swiglu_shift_ + kSwigluShiftStep);
            continue;
        }
        if (bits) throw_f16_range("forward", bits);
        break;
    }
    last_t_ = t_;
    return am;
}

uint32_t QwenExec::forward_chunks(int seq, int pos0, const int32_t* ids, int t_, float* logits, int logits_rows) {
    const QwenConfig& c = cfg_;
    uint32_t am = 0xFFFFFFFFu;
    // chunked prefill: max_tokens rows at a time, the cache carrying the earlier chunks
    for (int c0 = 0; c0 < t_; c0 += c.max_tokens) {
        const int n = std::min(c.max_tokens, t_ - c0);
        // the requested rows [t - logits_rows, t) that fall in this chunk: a suffix of it, `want` rows long, landing
        // at row `out0` of the caller's buffer
        const int first = std::max(c0, t_ - logits_rows);
        const int want = std::max(0, c0 + n - first);
        const int out0 = first - (t_ - logits_rows);
        std::vector<uint32_t> u(static_cast<size_t>(n));
        for (int i = 0; i < n; ++i) u[size_t(i)] = uint32_t(ids[c0 + i]);
        upload_tensor("ids", u.data(), uint64_t(n) * 4);
        // only the chunks holding some of the requested rows write into the caller's buffer
        float* lg = (logits && want > 0) ? logits + size_t(out0) * c.vocab : nullptr;
        if (c.mode == 1)
            am = forward_fast(seq, pos0 + c0, n, lg, std::max(want, 1));
        else
            am = forward_fp32(pos0 + c0, n, lg, std::max(want, 1));
    }
    return am;
}

void QwenExec::set_swiglu_shift(int s) {
    if (s == swiglu_shift_) return;
    swiglu_shift_ = s;
    if (decode_list_) {  // the recorded batched step carries the shift in its words
        dev_.release(decode_list_);
        decode_list_ = nullptr;
    }
}

void QwenExec::set_swiglu_shift_checked(int s) {
    if (cfg_.mode != 1) arg_fail("the SwiGLU shift is a fast-mode setting");
    if (s < 0 || s > kSwigluShiftLimit) arg_fail("SwiGLU shift %d outside 0 .. %d", s, kSwigluShiftLimit);
    set_swiglu_shift(s);
}

void QwenExec::throw_f16_range(const char* what, uint32_t bits) {
    throw RangeError(std::string(what) + ": a value stored as fp16 left the fp16 range (|x| > 65504, or NaN) at: " +
                     f16_range_sites(bits) + "; the results of this call are not usable");
}

uint32_t QwenExec::forward_fp32(int pos0, int T, float* logits, int lr) {
    const QwenConfig& c = cfg_;
    const uint32_t H = c.hidden, QC = c.heads * c.head_dim, KC = c.kv_heads * c.head_dim, I = c.intermediate,
                   V = c.vocab, HD = c.head_dim, U = uint32_t(T);
    const uint32_t eps = fbits(c.eps);
    const uint32_t scale = fbits(float(std::pow(double(HD), -0.5)));
    CommandList* l = dev_.begin();
    hipEvent_t e0, e1;
    hip_check(hipEventCreate(&e0), "event");
    hip_check(hipEventCreate(&e1), "event");
    auto tk = [&](const std::string& n) { return token(n); };
    dispatch(l, "embed_gather_bf16", {tk("ids"), tk("model.embed_tokens.weight"), tk("x"), U, H, V});
    tap_copy(l, "embed.out", tk("x"), T, int(H));
    for (int i = 0; i < c.layers; ++i) {
        std::string p = "L" + std::to_string(i) + ".";
        auto w = [&](int k) { return tk(lname(i, kLayerWeights[k])); };
        dispatch(l, "rmsnorm_rows", {tk("x"), w(0), tk("h"), U, H, eps});
        tap_copy(l, p + "input_layernorm.out", tk("h"), T, int(H));
        l->barrier();
        dispatch(l, "matmul_bf16w", {tk("h"), w(1), tk("q"), U, QC, H});
        dispatch(l, "matmul_bf16w", {tk("h"), w(2), tk("k"), U, KC, H});
        dispatch(l, "matmul_bf16w", {tk("h"), w(3), tk("v"), U, KC, H});
        tap_copy(l, p + "attn.q_proj.out", tk("q"), T, int(QC));
        tap_copy(l, p + "attn.k_proj.out", tk("k"), T, int(KC));
        tap_copy(l, p + "attn.v_proj.out", tk("v"), T, int(KC));
        l->barrier();
        dispatch(l, "rmsnorm_rows", {tk("q"), w(5), tk("qn"), U * c.heads, HD, eps});
        dispatch(l, "rmsnorm_rows", {tk("k"), w(6), tk("kn"), U * c.kv_heads, HD, eps});
        tap_copy(l, p + "attn.q_norm.out", tk("qn"), T, int(QC));
        tap_copy(l, p + "attn.k_norm.out", tk("kn"), T, int(KC));
        l->barrier();
        dispatch(l, "rope_apply", {tk("qn"), tk("rope.cos"), tk("rope.sin"), tk("qr"), U * c.heads, uint32_t(c.heads), HD, uint32_t(pos0)});
        dispatch(l, "rope_apply", {tk("kn"), tk("rope.cos"), tk("rope.sin"), tk("kr"), U * c.kv_heads, uint32_t(c.kv_heads), HD, uint32_t(pos0)});
        tap_copy(l, p + "attn.q_rope", tk("qr"), T, int(QC));
        tap_copy(l, p + "attn.k_rope", tk("kr"), T, int(KC));
        l->barrier();
        dispatch(l, "copy_rows", {tk("kr"), tk(p + "k_cache"), U, KC, 0, uint32_t(pos0), KC, KC});
        dispatch(l, "copy_rows", {tk("v"), tk(p + "v_cache"), U, KC, 0, uint32_t(pos0), KC, KC});
        if (c.taps) {
            TensorRow s = dev_.table().row(tk(p + "v_cache")), d = dev_.table().row(tk("tap." + p + "attn.v_cache"));
            l->copy(int(s.slot()), s.offset() + uint64_t(pos0) * KC * 4, int(d.slot()), d.offset(), uint64_t(T) * KC * 4);
        }
        l->barrier();
        dispatch(l, "attention_gqa_causal", {tk("qr"), tk(p + "k_cache"), tk(p + "v_cache"), tk("o"), U, 0,
                                             uint32_t(pos0), uint32_t(c.heads), uint32_t(c.kv_heads), HD, scale});
        tap_copy(l, p + "attn.o_proj.in", tk("o"), T, int(QC));
        l->barrier();
        dispatch(l, "matmul_bf16w", {tk("o"), w(4), tk("oo"), U, H, QC});
        tap_copy(l, p + "attn.o_proj.out", tk("oo"), T, int(H));
        l->barrier();
        dispatch(l, "add", {tk("x"), tk("oo"), tk("r"), U * H});
        tap_copy(l, p + "resid_mid", tk("r"), T, int(H));
        l->barrier();
        dispatch(l, "rmsnorm_rows", {tk("r"), w(7), tk("h2"), U, H, eps});
        tap_copy(l, p + "post_attention_layernorm.out", tk("h2"), T, int(H));
        l->barrier();
        dispatch(l, "matmul_bf16w", {tk("h2"), w(8), tk("g"), U, I, H});
        dispatch(l, "matmul_bf16w", {tk("h2"), w(9), tk("u"), U, I, H});
        tap_copy(l, p + "mlp.gate.out", tk("g"), T, int(I));
        tap_copy(l, p + "mlp.up.out", tk("u"), T, int(I));
        l->barrier();
        dispatch(l, "silu_mul", {tk("g"), tk("u"), tk("d"), U * I});
        tap_copy(l, p + "mlp.down.in", tk("d"), T, int(I));
        l->barrier();
        dispatch(l, "matmul_bf16w", {tk("d"), w(10), tk("dd"), U, H, I});
        tap_copy(l, p + "mlp.down.out", tk("dd"), T, int(H));
        l->barrier();
        dispatch(l, "add", {tk("r"), tk("dd"), tk("x"), U * H});
        tap_copy(l, p + "out", tk("x"), T, int(H));
        l->barrier();
    }
    dispatch(l, "rmsnorm_rows", {tk("x"), tk("model.norm.weight"), tk("f"), U, H, eps});
    tap_copy(l, "final_norm.out", tk("f"), T, int(H));
    l->barrier();
    const uint32_t LR = uint32_t(c.taps ? T : lr);
    if (LR > dev_.table().row(tk("logits")).count() / V) arg_fail("%u logits rows exceed the logits tensor", LR);
    dispatch(l, "copy_rows", {tk("f"), tk("f_last"), LR, H, U - LR, 0, H, H});
    l->barrier();
    dispatch(l, "matmul_bf16w", {tk("f_last"), tk("model.embed_tokens.weight"), tk("logits"), LR, V, H});
    if (c.taps) tap_copy(l, "logits", tk("logits"), T, int(V));
    l->barrier();
    dispatch(l, "argmax_rows", {tk("logits"), tk("argmax"), LR, V});
    hip_check(hipEventRecord(e0, dev_.stream()), "event");
    uint64_t f = dev_.submit(l);
    hip_check(hipEventRecord(e1, dev_.stream()), "event");
    dev_.wait(f);
    dev_.release(l);
    hip_check(hipEventSynchronize(e1), "event");
    float ms = 0;
    hip_check(hipEventElapsedTime(&ms, e0, e1), "event");
    last_ms_ = ms;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (logits) download_tensor("logits", logits, uint64_t(lr) * V * 4, uint64_t(LR - uint32_t(lr)) * V * 4);
    uint32_t am = 0;
    download_tensor("argmax", &am, 4, uint64_t(LR - 1) * 4);
    return am;
}

// The k splits of a prefill residual GEMM of m rows (128 x 64 output tiles): the fewest of 1, 2, 4 that give at least
// 512 blocks (two per CU), within the partials tensor (2 max_tokens rows) and with k a multiple of 64 per split. Not 8:
// at 512 rows (64 tiles) 8 splits leave each block 4-6 k steps and the add pass 8 partials to read, and the 512-token
// forward measured 2.53 ms against 2.40 ms with 4.
// Row widths residual_add_norm (one wave per row, 256-column steps) takes; other hidden sizes run the residual GEMM
// and a separate norm.
static bool add_norm_width(uint32_t n) { return n == 256 || n == 512 || n == 1024 || n == 2048 || n == 4096; }

static uint32_t resid_splits(uint32_t m, uint32_t n, uint32_t k, uint32_t max_tokens) {
    if (!add_norm_width(n)) return 1;
    const uint64_t tiles = uint64_t((n + 63) / 64) * ((m + 127) / 128);
    // up to 512 rows the GEMM runs 64-row tiles, and two splits then fill the CUs with half the partials for
    // residual_add_norm to add (512-token forward: 2.27 -> 2.24 ms against four splits of 128-row tiles)
    const uint32_t smax = m <= 512 ? 2 : 4;
    uint32_t s = 1;
    while (s < smax && tiles * s < 512 && 2 * s * m <= 2 * max_tokens && k % (128 * s) == 0) s *= 2;
    return s;
}

uint32_t QwenExec::forward_fast(int seq, int pos0, int T, float* logits, int lr) {
    const std::string sq = ".s" + std::to_string(seq);
    const QwenConfig& c = cfg_;
    const uint32_t H = c.hidden, QC = c.heads * c.head_dim, I = c.intermediate, V = c.vocab, HD = c.head_dim,
                   MP = c.max_pos, U = uint32_t(T);
    const uint32_t eps = fbits(c.eps);
    const uint32_t scale = fbits(float(std::pow(double(HD), -0.5)));
    auto tk = [&](const std::string& n) { return token(n); };
    const uint32_t LC = dev_.table().row(tk("logits")).count() / V;
    const uint32_t ash = uint32_t(swiglu_shift_);
    sync_f16();
    CommandList* l = dev_.begin();
    dispatch(l, "embed_gather_bf16", {tk("ids"), tk("model.embed_tokens.weight"), tk("x"), U, H, V});
    // x += a . W^T, then h = RMSNorm(x) with norm weights nw: a k-split GEMM into partials and one pass that adds them
    // and normalises (the split fills the CUs: at 2048 rows the 128 x 64 tiles alone give one block per CU), or, with no
    // split, the residual GEMM and the norm
    const uint32_t MT = uint32_t(c.max_tokens);
    auto residual_norm = [&](const std::string& a, const std::string& wname, uint32_t K, uint32_t nw, uint32_t sh) {
        const uint32_t sp = resid_splits(U, H, K, MT);
        if (sp > 1) {
            dispatch(l, "gemm_residual_split", {tk(a), tk(wname), tk("resid.partials"), U, H, K, sp, sh});
            dispatch(l, "residual_add_norm", {tk("x"), tk("resid.partials"), nw, tk("h"), U, H, sp, eps});
        } else {
            dispatch(l, "gemm_residual", {tk(a), tk(wname), tk("x"), U, H, K, sh});
            dispatch(l, "rmsnorm_rows_f16", {tk("x"), nw, tk("h"), U, H, eps, 0});
        }
    };
    dispatch(l, "rmsnorm_rows_f16", {tk("x"), tk(lname(0, kLayerWeights[0])), tk("h"), U, H, eps, 0});
    for (int i = 0; i < c.layers; ++i) {
        const std::string p = "L" + std::to_string(i) + ".";
        auto w = [&](int k) { return tk(lname(i, kLayerWeights[k])); };
        // h = RMSNorm(x) with this layer's input norm: done by the previous layer's down_proj step (or above)
        dispatch(l, "gemm_qkv_rope", {tk("h"), tk(p + "qkv_proj.f16"), w(5), w(6), tk("rope.cos"), tk("rope.sin"),
                                      tk("q"), tk(p + "k_cache" + sq), tk(p + "v_cache" + sq), U, H,
                                      uint32_t(c.heads), uint32_t(c.kv_heads), uint32_t(pos0), MP, eps});
        dispatch(l, "attention_prefill_f16", {tk("q"), tk(p + "k_cache" + sq), tk(p + "v_cache" + sq), tk("o"),
                                              tk("attn.ws"), U, uint32_t(pos0), uint32_t(c.heads),
                                              uint32_t(c.kv_heads), MP, scale});
        residual_norm("o", p + "o_proj.f16", QC, w(7), 0);
        dispatch(l, "gemm_swiglu", {tk("h"), tk(p + "gate_up_proj.f16"), tk("a"), U, I, H, ash});
        // the next layer's input norm (after the last layer: the final norm, which the lm_head pass below recomputes
        // on its rows)
        residual_norm("a", p + "down_proj.f16", I,
                      i + 1 < c.layers ? tk(lname(i + 1, kLayerWeights[0])) : tk("model.norm.weight"), ash);
    }
    // logits of the last lr rows, LC rows per lm_head dispatch: the final norm over rows r0 .. r0 + n - 1, the lm_head
    // GEMM, and after the last rows the argmax of the last one (the forward returns the last row's id)
    auto lm_head = [&](CommandList* L, int r0, uint32_t n) {
        dispatch(L, "rmsnorm_rows_f16", {tk("x"), tk("model.norm.weight"), tk("h"), n, H, eps, uint32_t(r0)});
        dispatch(L, "gemm_f32", {tk("h"), tk("embed.f16"), tk("logits"), n, V, H});
        if (r0 + int(n) == T) {
            dispatch(L, "argmax_rows_partial", {tk("logits"), tk("argmax.partials"), 1, V, n - 1});
            dispatch(L, "argmax_rows_final", {tk("argmax.partials"), tk("argmax"), 1});
        }
    };
    // rows that fit one dispatch ride in the layers' list: one submission, so the GPU does not wait for the host
    // between the last layer and the lm_head (2048-token prefill, last row: 4.11 -> 4.09 ms; 512-token forward with
    // all its logits: 2.22 -> 2.19 ms)
    const bool one = uint32_t(lr) <= LC;
    if (one) lm_head(l, T - lr, uint32_t(lr));
    hipEvent_t e0, e1;
    hip_check(hipEventCreate(&e0), "event");
    hip_check(hipEventCreate(&e1), "event");
    hip_check(hipEventRecord(e0, dev_.stream()), "event");
    uint64_t f = dev_.submit(l);
    if (one) hip_check(hipEventRecord(e1, dev_.stream()), "event");
    dev_.wait(f);
    dev_.release(l);
    uint32_t am = 0;
    if (one) {
        hip_check(hipEventSynchronize(e1), "event");
        download_tensor("argmax", &am, 4, 0);
        if (logits) download_tensor("logits", logits, uint64_t(lr) * V * 4);
    }
    for (int r0 = T - lr; !one && r0 < T; r0 += int(LC)) {
        const uint32_t n = uint32_t(std::min(int(LC), T - r0));
        CommandList* l2 = dev_.begin();
        lm_head(l2, r0, n);
        uint64_t f2 = dev_.submit(l2);
        dev_.wait(f2);
        dev_.release(l2);
        const bool last = r0 + int(n) == T;
        if (last) {
            hip_check(hipEventRecord(e1, dev_.stream()), "event");
            hip_check(hipEventSynchronize(e1), "event");
            download_tensor("argmax", &am, 4, 0);
        }
        if (logits) download_tensor("logits", logits + size_t(r0 - (T - lr)) * V, uint64_t(n) * V * 4);
    }
    float ms = 0;
    hip_check(hipEventElapsedTime(&ms, e0, e1), "event");
    last_ms_ = ms;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return am;
}

// ---------------------------------------------------------------- decode (fast mode)
// One step: embed the fed-back token; per layer the fused q|k|v GEMV on RMSNorm(x), split-KV attention (q/k norm,
// RoPE and the cache append inside), the split combine, o_proj + residual, the SwiGLU GEMV pair on RMSNorm(x), down +
// residual; then the lm_head partial argmaxes and the final argmax, which advances the on-device state.

void QwenExec::record_decode_fast() {
    const QwenConfig& c = cfg_;
    const uint32_t H = c.hidden, QC = c.heads * c.head_dim, KC = c.kv_heads * c.head_dim, I = c.intermediate,
                   V = c.vocab, HD = c.head_dim, MP = c.max_pos;
    const uint32_t eps = fbits(c.eps);
    const uint32_t scale = fbits(float(std::pow(double(HD), -0.5)));
    auto tk = [&](const std::string& n) { return token(n); };
    CommandList* l = dev_.begin(true);
    const uint32_t B = uint32_t(c.batch);
    if (B > 1) {
        record_decode_batch(l);
        decode_list_ = l;
        return;
    }
    if (persist_) {
        dispatch(l, "decode_step_persistent",
                 {tk("model.embed_tokens.weight"), tk("model.norm.weight"), tk("stack.input_layernorm"),
                  tk("stack.qkv_proj.f16"), tk("stack.q_norm"), tk("stack.k_norm"), tk("stack.o_proj.f16"),
                  tk("stack.post_attention_layernorm"), tk("stack.gate_up_proj.f16"), tk("stack.down_proj.f16"),
                  tk("stack.k_cache"), tk("stack.v_cache"), tk("rope.cos"), tk("rope.sin"), tk("logits"), tk("dec.state"),
                  tk("dec.out_ids"), tk("dec.exchange"), tk("embed.f16"), uint32_t(c.layers), H, uint32_t(c.heads),
                  uint32_t(c.kv_heads), I, V, MP, MP, 1, eps, scale, uint32_t(persist_blocks_)});
        decode_list_ = l;
        return;
    }
    dispatch(l, "embed_dec", {tk("model.embed_tokens.weight"), tk("dec.state"), tk("dec.x"), H, V, 1});
    for (int i = 0; i < c.layers; ++i) {
        const std::string p = "L" + std::to_string(i) + ".";
        auto w = [&](int k) { return tk(lname(i, kLayerWeights[k])); };
        dispatch(l, "gemv_norm_dec", {tk("dec.x"), w(0), tk(p + "qkv_proj"), tk("dec.qkv"), QC + 2 * KC, H, eps});
        dispatch(l, "attention_decode_f16", {tk("dec.qkv"), w(5), w(6), tk("rope.cos"), tk("rope.sin"),
                                             tk(p + "k_cache"), tk(p + "v_cache"), tk("dec.attn_partials"),
                                             tk("dec.state"), uint32_t(c.heads), uint32_t(c.kv_heads), MP, eps, scale,
                                             1});
        dispatch(l, "attention_combine", {tk("dec.attn_partials"), tk("dec.o"), tk("dec.state"), uint32_t(c.heads), MP,
                                          1});
        dispatch(l, "gemv_residual_dec", {tk("dec.o"), w(4), tk("dec.x"), H, QC});
        dispatch(l, "gemv_swiglu_dec", {tk("dec.x"), w(7), tk(p + "gate_up_proj"), tk("dec.a"), I, H, eps});
        dispatch(l, "gemv_residual_dec", {tk("dec.a"), w(10), tk("dec.x"), H, I});
    }
    dispatch(l, "lmhead_dec", {tk("dec.x"), tk("model.norm.weight"), tk("model.embed_tokens.weight"), tk("logits"),
                               tk("dec.lm_partials"), V, H, eps, 1});
    dispatch(l, "argmax_dec", {tk("dec.lm_partials"), tk("dec.state"), tk("dec.out_ids"), MP});
    decode_list_ = l;
}

// One batched step (B > 1): embed; per layer RMSNorm -> fp16 rows, the q|k|v skinny GEMM, split-KV attention per
// sequence (norm, RoPE and the cache append inside), the combine (fp16 out), o_proj + residual, RMSNorm, the gate/up
// SwiGLU GEMM, down + residual; then the final norm, the lm_head GEMM over the B rows, the split argmax and the state
// advance.
void QwenExec::record_decode_batch(CommandList* l) {
    const QwenConfig& c = cfg_;
    const uint32_t H = c.hidden, QC = c.heads * c.head_dim, KC = c.kv_heads * c.head_dim, I = c.intermediate,
                   V = c.vocab, HD = c.head_dim, MP = c.max_pos, B = uint32_t(c.batch);
    const uint32_t eps = fbits(c.eps);
    const uint32_t scale = fbits(float(std::pow(double(HD), -0.5)));
    // decode-attention splits per (sequence, KV head): one multi-chunk block per CU (measured at 16 sequences x 8K,
    // 1.7B: 2 splits 4.03 ms per step, 4 splits, i.e. two blocks per CU, 4.09, 8 splits 4.09, 3 splits 4.27); each
    // sequence's keys spread evenly over its splits (sized on the device from its position), so the blocks finish
    // together instead of leaving a partly filled last round
    const uint32_t pairs = B * uint32_t(c.kv_heads);
    const uint32_t splits = std::min(MP / 64, std::max(1u, uint32_t(dev_.info().compute_units) / pairs));
    auto tk = [&](const std::string& n) { return token(n); };
    // x += a . W^T, then h = RMSNorm(x) with norm weights nw: the GEMM split over k in two (twice the blocks: one
    // block per 16 columns alone leaves half the CUs idle at hidden 2048) into partials, then one pass that adds them
    // and normalises; or, when k does not split in 1024-multiples, the residual GEMM and the norm
    const uint32_t ash = uint32_t(swiglu_shift_);
    auto residual_norm = [&](const std::string& a, const std::string& wname, uint32_t K, uint32_t nw, uint32_t sh) {
        if (K % 2048 == 0 && add_norm_width(H)) {
            dispatch(l, "gemm_residual_split", {tk(a), tk(wname), tk("resid.partials"), B, H, K, 2, sh});
            dispatch(l, "residual_add_norm", {tk("dec.x"), tk("resid.partials"), nw, tk("dec.h16"), B, H, 2, eps});
        } else {
            dispatch(l, "gemm_skinny_residual", {tk(a), tk(wname), tk("dec.x"), B, H, K, sh});
            dispatch(l, "rmsnorm_rows_f16", {tk("dec.x"), nw, tk("dec.h16"), B, H, eps, 0});
        }
    };
    dispatch(l, "embed_dec", {tk("model.embed_tokens.weight"), tk("dec.state"), tk("dec.x"), H, V, B});
    dispatch(l, "rmsnorm_rows_f16", {tk("dec.x"), tk(lname(0, kLayerWeights[0])), tk("dec.h16"), B, H, eps, 0});
    for (int i = 0; i < c.layers; ++i) {
        const std::string p = "L" + std::to_string(i) + ".";
        auto w = [&](int k) { return tk(lname(i, kLayerWeights[k])); };
        // h = RMSNorm(x) with this layer's input norm: done above or by the previous layer's down_proj step
        dispatch(l, "gemm_skinny_f32", {tk("dec.h16"), tk(p + "qkv_proj.f16"), tk("dec.qkv"), B, QC + 2 * KC, H});
        dispatch(l, "attention_decode_f16", {tk("dec.qkv"), w(5), w(6), tk("rope.cos"), tk("rope.sin"),
                                             tk(p + "k_cache"), tk(p + "v_cache"), tk("dec.attn_partials"),
                                             tk("dec.state"), uint32_t(c.heads), uint32_t(c.kv_heads), MP, eps, scale,
                                             B, 0, splits});
        dispatch(l, "attention_combine_f16", {tk("dec.attn_partials"), tk("dec.o16"), tk("dec.state"),
                                              uint32_t(c.heads), MP, B, 0, splits});
        residual_norm("dec.o16", p + "o_proj.f16", QC, w(7), 0);
        dispatch(l, "gemm_skinny_swiglu", {tk("dec.h16"), tk(p + "gate_up_proj.f16"), tk("dec.a16"), B, I, H, ash});
        // the next layer's input norm (after the last layer: the final norm, the lm_head's input)
        residual_norm("dec.a16", p + "down_proj.f16", I,
                      i + 1 < c.layers ? tk(lname(i + 1, kLayerWeights[0])) : tk("model.norm.weight"), ash);
    }
    dispatch(l, "gemm_skinny_f32", {tk("dec.h16"), tk("embed.f16"), tk("logits"), B, V, H});
    dispatch(l, "argmax_rows_partial", {tk("logits"), tk("argmax.partials"), B, V});
    dispatch(l, "argmax_rows_final", {tk("argmax.partials"), tk("argmax"), B});
    dispatch(l, "decode_advance", {tk("argmax"), tk("dec.state"), tk("dec.out_ids"), B, MP});
}

void QwenExec::set_decode_state(const int32_t* ids, const int32_t* pos) {
    if (cfg_.mode != 1) arg_fail("on-device decode needs the fast mode");
    const int B = cfg_.batch;
    std::vector<uint32_t> st(size_t(2 * B + 2), 0u);
    for (int b = 0; b < B; ++b) {
        if (pos[b] < 0 || pos[b] >= cfg_.max_pos) arg_fail("decode position %d outside max_pos %d", pos[b], cfg_.max_pos);
        st[size_t(b)] = uint32_t(pos[b]);
        st[size_t(B + b)] = uint32_t(ids[b]);
    }
    upload_tensor("dec.state", st.data(), st.size() * 4);
    if (persist_) {
        // After an aborted step the exchange entries are in an unknown mix of steps: start over from zeros (epoch 0,
        // every entry untagged); otherwise the entries of the last step carry its tag, which the next launch's differs
        // from. LRM_HIP_PERSIST_WAIT_US bounds each wait of the step's workgroups (default 0.2 s): a tiny bound makes
        // steps abort, which is how the failure path is tested.
        uint32_t hdr[4];
        download_tensor("dec.exchange", hdr, sizeof hdr);
        if (hdr[1]) {
            std::vector<uint8_t> zero(dev_.table().row(token("dec.exchange")).extent_bytes(), 0);
            upload_tensor("dec.exchange", zero.data(), zero.size());
            hdr[0] = hdr[1] = hdr[2] = 0u;
        }
        const char* w = std::getenv("LRM_HIP_PERSIST_WAIT_US");
        const long us = w ? std::strtol(w, nullptr, 10) : 0;
        hdr[3] = us > 0 ? uint32_t(std::min<long>(us, 40000000L) * 100) : 0u;
        upload_tensor("dec.exchange", hdr, sizeof hdr);
    }
}

void QwenExec::run_decode_steps(int steps) {
    if (cfg_.mode != 1) arg_fail("on-device decode needs the fast mode");
    if (steps < 1) return;
    const int B = cfg_.batch;
    std::vector<uint32_t> st(size_t(2 * B + 2));
    download_tensor("dec.state", st.data(), st.size() * 4);
    for (int b = 0; b < B; ++b)
        if (int64_t(st[size_t(b)]) + steps > cfg_.max_pos)
            arg_fail("%d decode steps from position %u pass max_pos %d", steps, st[size_t(b)], cfg_.max_pos);
    if (!decode_list_) record_decode_fast();
    sync_f16();  // the batched step's skinny GEMMs read the fp16 copies: weights set since the last forward
    hipEvent_t e0, e1;
    hip_check(hipEventCreate(&e0), "event");
    hip_check(hipEventCreate(&e1), "event");
    hip_check(hipEventRecord(e0, dev_.stream()), "event");
    uint64_t f = dev_.submit(decode_list_, uint32_t(steps));
    hip_check(hipEventRecord(e1, dev_.stream()), "event");
    dev_.wait(f);
    hip_check(hipEventSynchronize(e1), "event");
    float ms = 0;
    hip_check(hipEventElapsedTime(&ms, e0, e1), "event");
    last_ms_ = ms;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (persist_) {  // a workgroup that waited past its bound aborted the step (and every later one)
        uint32_t hdr[3];
        download_tensor("dec.exchange", hdr, sizeof hdr);
        if (hdr[1] && hdr[2] == uint32_t(persist::kStageClaim))
            throw std::runtime_error("decode_step_persistent: two workgroups of one launch took the same (XCD, role) "
                                     "slot (the dispatcher placed the workgroups otherwise than the step assumes); "
                                     "the step's results are not valid");
        if (hdr[1])
            throw std::runtime_error("decode_step_persistent: a workgroup waited past its bound at stage " +
                                     std::to_string(hdr[2]) + "; the decode state did not advance from there");
    }
    // A decode call cannot rerun (its steps advanced the state): it fails, and a SwiGLU overflow raises the shift
    // for the calls after it.
    const uint32_t bits = dev_.take_f16_range();
    if (bits & kF16SiteSwiglu) set_swiglu_shift(std::min(kMaxSwigluShift, swiglu_shift_ + kSwigluShiftStep));
    if (bits) throw_f16_range("decode", bits);
}

void QwenExec::read_decode_ids(int32_t* out, int count) {
    if (count < 0 || int64_t(count) > int64_t(cfg_.max_pos) * cfg_.batch) arg_fail("count %d", count);
    download_tensor("dec.out_ids", out, uint64_t(count) * 4);
}

void QwenExec::greedy(const int32_t* prompt, int plen, int steps, int32_t* out) {
    const QwenConfig& c = cfg_;
    if (plen < 1 || steps < 1) arg_fail("greedy: empty prompt or no steps");
    if (c.batch != 1) arg_fail("greedy decodes one sequence: use decode_batch for %d", c.batch);
    if (plen + steps - 1 > c.max_pos) arg_fail("greedy: %d positions exceed max_pos %d", plen + steps - 1, c.max_pos);
    uint32_t id = forward(0, 0, prompt, plen, nullptr, 1);
    if (id == 0xFFFFFFFFu) throw std::runtime_error("greedy: argmax of a row that holds a NaN");
    out[0] = int32_t(id);
    if (steps == 1) return;
    if (c.mode == 1) {
        int32_t pos = plen;
        int32_t i0 = int32_t(id);
        set_decode_state(&i0, &pos);
        uint32_t st[4] = {uint32_t(plen), id, 1, 0};
        upload_tensor("dec.state", st, 16);
        run_decode_steps(steps - 1);
        std::vector<int32_t> ids(static_cast<size_t>(steps));
        read_decode_ids(ids.data(), steps);
        for (int s = 1; s < steps; ++s) {
            if (uint32_t(ids[size_t(s)]) == 0xFFFFFFFFu) throw std::runtime_error("greedy: argmax of a row that holds a NaN");
            out[s] = ids[size_t(s)];
        }
        return;
    }
    for (int s = 1; s < steps; ++s) {
        int32_t cur = out[s - 1];
        uint32_t nx = forward(0, plen + s - 1, &cur, 1, nullptr, 1);
        if (nx == 0xFFFFFFFFu) throw std::runtime_error("greedy: argmax of a row that holds a NaN");
        out[s] = int32_t(nx);
    }
}

void QwenExec::decode_batch(const int32_t* ids, const int32_t* pos, int steps, int32_t* out_ids) {
    if (steps < 1) arg_fail("decode_batch: no steps");
    set_decode_state(ids, pos);
    run_decode_steps(steps);
    read_decode_ids(out_ids, steps * cfg_.batch);
}

// ---------------------------------------------------------------- taps and caches

int QwenExec::tap_count() const { return int(tap_names_.size()); }
std::string QwenExec::tap_name(int i) const { return tap_names_.at(size_t(i)); }
int QwenExec::tap_width(int i) const { return tap_widths_.at(size_t(i)); }

void QwenExec::read_tap(int i, float* out, int rows) {
    if (i < 0 || i >= tap_count()) arg_fail("tap %d of %d", i, tap_count());
    if (rows < 0 || rows > cfg_.max_tokens) arg_fail("tap rows %d", rows);
    download_tensor("tap." + tap_names_[size_t(i)], out, uint64_t(rows) * tap_widths_[size_t(i)] * 4);
}

// IEEE binary16 <-> binary32 on the host (round to nearest even), for the fp16 caches of the fast mode.
static float half_to_float(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t u;
    if (e == 0x1F) {
        u = sign | 0x7F800000u | (m << 13);
    } else if (e == 0) {
        u = sign | fbits(float(m) * 0x1p-24f);  // zero or a subnormal: m * 2^-24 is exact in binary32
    } else {
        u = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

static uint16_t float_to_half(float f) {
    const uint32_t u = fbits(f), sign = (u >> 16) & 0x8000u, a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return uint16_t(sign | 0x7E00u);  // NaN
    if (a >= 0x477FF000u) return uint16_t(sign | 0x7C00u);  // at or past 65520, the midpoint to infinity
    if (a <= 0x33000000u) return uint16_t(sign);            // at or below 2^-25, the midpoint to the least subnormal
    const int e = int(a >> 23) - 127;
    const uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
    uint32_t q, rem, half;
    if (e < -14) {  // subnormal result: units of 2^-24
        const int sh = -1 - e;  // 14 .. 24
        q = m >> sh;
        rem = m & ((1u << sh) - 1);
        half = 1u << (sh - 1);
    } else {
        q = (uint32_t(e + 15) << 10) | ((m >> 13) & 0x3FFu);
        rem = m & 0x1FFFu;
        half = 0x1000u;
    }
    if (rem > half || (rem == half && (q & 1u))) ++q;  // a carry into the exponent field is the right result
    return uint16_t(sign | q);
}

void QwenExec::read_cache(int seq, int layer, int which, int row0, int rows, float* out) {
    const QwenConfig& c = cfg_;
    if (seq < 0 || seq >= c.batch || layer < 0 || layer >= c.layers || row0 < 0 || rows < 0 || row0 + rows > c.max_pos)
        arg_fail("cache rows out of range");
    const int KC = c.kv_heads * c.head_dim, HD = c.head_dim, MP = c.max_pos;
    std::string n = "L" + std::to_string(layer) + (which ? ".v_cache" : ".k_cache");
    if (c.mode == 0) {
        download_tensor(n, out, uint64_t(rows) * KC * 4, uint64_t(row0) * KC * 4);
        return;
    }
    n += ".s" + std::to_string(seq);  // this sequence's heads
    std::vector<uint16_t> all(size_t(c.kv_heads) * MP * HD);
    download_tensor(n, all.data(), all.size() * 2);
    for (int r = 0; r < rows; ++r)
        for (int h = 0; h < c.kv_heads; ++h)
            for (int d = 0; d < HD; ++d) {
                size_t src = which ? size_t(h) * HD * MP + kv::v_at(row0 + r, d) : (size_t(h) * MP + row0 + r) * HD + d;
                out[size_t(r) * KC + h * HD + d] = half_to_float(all[src]);
            }
}

void QwenExec::write_cache(int seq, int layer, int which, int row0, int rows, const float* in) {
    const QwenConfig& c = cfg_;
    if (seq < 0 || seq >= c.batch || layer < 0 || layer >= c.layers || row0 < 0 || rows < 0 || row0 + rows > c.max_pos)
        arg_fail("cache rows out of range");
    const int KC = c.kv_heads * c.head_dim, HD = c.head_dim, MP = c.max_pos;
    std::string n = "L" + std::to_string(layer) + (which ? ".v_cache" : ".k_cache");
    if (c.mode == 0) {
        upload_tensor(n, in, uint64_t(rows) * KC * 4, uint64_t(row0) * KC * 4);
        return;
    }
    n += ".s" + std::to_string(seq);  // this sequence's heads
    std::vector<uint16_t> all(size_t(c.kv_heads) * MP * HD);
    download_tensor(n, all.data(), all.size() * 2);
    for (int r = 0; r < rows; ++r)
        for (int h = 0; h < c.kv_heads; ++h)
            for (int d = 0; d < HD; ++d) {
                size_t dst = which ? size_t(h) * HD * MP + kv::v_at(row0 + r, d) : (size_t(h) * MP + row0 + r) * HD + d;
                all[dst] = float_to_half(in[size_t(r) * KC + h * HD + d]);
            }
    upload_tensor(n, all.data(), all.size() * 2);
}

void QwenExec::fill_cache_random(uint64_t seed, int rows) {
    const QwenConfig& c = cfg_;
    if (c.mode != 1) arg_fail("fill_cache_random needs the fp16 cache of the fast mode");
    if (rows < 0 || rows > c.max_pos) arg_fail("rows %d", rows);
    // Whole caches are filled (positions past `rows` are never read before they are written).
    CommandList* l = dev_.begin();
    float one = 1.0f;
    for (int i = 0; i < c.layers; ++i)
        for (int which = 0; which < 2; ++which) {
            std::string n = "L" + std::to_string(i) + (which ? ".v_cache" : ".k_cache");
            uint32_t cnt = dev_.table().row(token(n)).count();
            uint64_t st = stream_of(n.c_str());
            dispatch(l, "fill_normal_f16", {token(n), cnt, uint32_t(seed), uint32_t(seed >> 32), uint32_t(st),
                                             uint32_t(st >> 32), fbits(one)});
        }
    dev_.wait(dev_.submit(l));
    dev_.release(l);
}

}  // namespace lrm
