// extern "C" entry points of liblrm_hip.so (include/lrm_hip.h): thin wrappers that map C++ exceptions to status codes
// and a thread-local message.
#include <algorithm>
#include <cctype>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>

#include "../../include/lrm_hip.h"
#include "contract.hpp"
#include "device.hpp"
#include "qwen_exec.hpp"
#include "safetensors.hpp"
#include "tokenizer.hpp"

using namespace lrm;

static thread_local std::string g_err;

template <class F>
static int guard(F&& f) {
    try {
        f();
        return LRM_OK;
    } catch (const ContractError& e) {
        g_err = e.what();
        return LRM_E_CONTRACT;
    } catch (const HipError& e) {
        g_err = e.what();
        return LRM_E_HIP;
    } catch (const RangeError& e) {
        g_err = e.what();
        return LRM_E_RANGE;
    } catch (const FormatError& e) {
        g_err = e.what();
        return LRM_E_FORMAT;
    } catch (const IntegrityError& e) {
        g_err = e.what();
        return LRM_E_INTEGRITY;
    } catch (const tok::DataError& e) {
        g_err = e.what();
        return LRM_E_DATA;
    } catch (const std::out_of_range& e) {
        g_err = e.what();
        return LRM_E_ARG;
    } catch (const std::invalid_argument& e) {
        g_err = e.what();
        return LRM_E_ARG;
    } catch (const std::exception& e) {
        g_err = e.what();
        return LRM_E_INTERNAL;
    } catch (...) {
        g_err = "unknown failure";
        return LRM_E_INTERNAL;
    }
}

static void need_ptr(const void* p, const char* what) {
    if (!p) throw std::invalid_argument(std::string(what) + " is NULL");
}

static void copy_str(char* dst, int cap, const char* src) {
    if (!dst || cap <= 0) return;
    std::snprintf(dst, size_t(cap), "%s", src);
}

static HeapLayout layout_of(const uint32_t* arenas, const uint64_t* bytes, int pages) {
    if (pages < 0 || (pages > 0 && (!arenas || !bytes))) throw std::invalid_argument("bad page list");
    std::vector<std::pair<uint32_t, uint64_t>> kb;
    for (int i = 0; i < pages; ++i) kb.emplace_back(arenas[i], bytes[i]);
    return HeapLayout::of_pages(kb);
}

struct lrm_planner {
    HeapPlanner p;
};
struct lrm_table {
    TensorTable t;
};
struct lrm_hip_device {
    Device d;
    lrm_hip_device(int index, uint32_t flags) : d(index, flags) {}
};
struct lrm_hip_list {
    CommandList* l;
    lrm_hip_device* owner;
};
struct lrm_qwen {
    QwenExec q;
    lrm_hip_device* dev;
    lrm_qwen(lrm_hip_device* d, const QwenConfig& c, const uint32_t* inv) : q(d->d, c, inv), dev(d) {}
};

// Copies `n` items to `out` when they fit in `cap` (nothing otherwise); *count = n either way.
template <class T>
static void fill_out(const T* src, size_t n, T* out, uint64_t cap, uint64_t* count) {
    need_ptr(count, "count");
    *count = n;
    if (out && cap >= n && n) std::memcpy(out, src, n * sizeof(T));
}

extern "C" {

const char* lrm_last_error(void) { return g_err.c_str(); }
int lrm_abi_version(void) { return LRM_ABI_VERSION; }

// ---------------------------------------------------------------- contract helpers

int lrm_catalog_count(void) { return catalog_size(); }
int lrm_catalog_find(const char* name) { return name ? catalog_find(name) : -1; }

int lrm_catalog_kernel(uint32_t id, char* name, int cap, uint32_t threads[3], int* linear, int* field_count) {
    return guard([&] {
        if (id >= uint32_t(catalog_size())) contract_fail("kernel id %u is not in the catalog", id);
        const KernelSpec& k = catalog()[id];
        copy_str(name, cap, k.name);
        if (threads)
            for (int i = 0; i < 3; ++i) threads[i] = uint32_t(k.threads[i]);
        if (linear) *linear = k.linear;
        if (field_count) *field_count = int(k.fields.size());
    });
}

int lrm_catalog_field(uint32_t id, int field, char* name, int cap, int* kind, int* access, uint32_t* mask) {
    return guard([&] {
        if (id >= uint32_t(catalog_size())) contract_fail("kernel id %u is not in the catalog", id);
        const KernelSpec& k = catalog()[id];
        if (field < 0 || field >= int(k.fields.size())) contract_fail("kernel %s has no field %d", k.name, field);
        const FieldSpec& f = k.fields[size_t(field)];
        copy_str(name, cap, f.name);
        if (kind) *kind = int(f.kind);
        if (access) *access = int(f.access);
        if (mask) *mask = f.dtype_mask;
    });
}

int lrm_grid_physical(int linear, int64_t x, int64_t y, int64_t z, uint32_t out[3]) {
    return guard([&] {
        need_ptr(out, "out");
        Physical p = grid_physical(linear != 0, Grid3{x, y, z});
        out[0] = p.x;
        out[1] = p.y;
        out[2] = p.z;
    });
}

int lrm_tensor_row(int slot, uint64_t off, uint32_t dtype, const uint32_t* dims, int rank, uint32_t flags,
                   const char* name, uint32_t out[16]) {
    return guard([&] {
        need_ptr(out, "out");
        if (rank < 0 || (rank > 0 && !dims)) throw std::invalid_argument("bad dims");
        TensorRow r = TensorRow::create(slot, off, dtype, std::vector<uint32_t>(dims, dims + rank), flags, name ? name : "");
        std::memcpy(out, r.w.data(), 64);
    });
}

uint32_t lrm_debug_id(const char* name) { return debug_id_of(name ? name : ""); }

int lrm_planner_create(uint64_t page_bytes, lrm_planner** out) {
    return guard([&] {
        need_ptr(out, "out");
        *out = new lrm_planner{HeapPlanner(page_bytes)};
    });
}

int lrm_planner_allocate(lrm_planner* p, uint32_t arena, uint64_t bytes, int32_t* page, uint64_t* offset) {
    return guard([&] {
        need_ptr(p, "planner");
        Placement pl = p->p.allocate(arena, bytes);
        if (page) *page = pl.page;
        if (offset) *offset = pl.offset;
    });
}

int lrm_planner_build(lrm_planner* p, uint32_t* arenas, uint64_t* bytes, int cap, int* pages) {
    return guard([&] {
        need_ptr(p, "planner");
        HeapLayout l = p->p.build();
        if (pages) *pages = int(l.pages.size());
        for (size_t i = 0; i < l.pages.size() && int(i) < cap; ++i) {
            if (arenas) arenas[i] = l.pages[i].arena;
            if (bytes) bytes[i] = l.pages[i].bytes;
        }
    });
}

void lrm_planner_destroy(lrm_planner* p) { delete p; }

int lrm_table_create(const uint32_t* arenas, const uint64_t* bytes, int pages, lrm_table** out) {
    return guard([&] {
        need_ptr(out, "out");
        *out = new lrm_table{TensorTable(layout_of(arenas, bytes, pages))};
    });
}

int lrm_table_add(lrm_table* t, const char* name, int slot, uint64_t off, uint32_t dtype, const uint32_t* dims, int rank,
                  uint32_t flags, uint32_t* token) {
    return guard([&] {
        need_ptr(t, "table");
        if (rank < 0 || (rank > 0 && !dims)) throw std::invalid_argument("bad dims");
        uint32_t tok = t->t.add(name ? name : "", slot, off, dtype, std::vector<uint32_t>(dims, dims + rank), flags);
        if (token) *token = tok;
    });
}

int lrm_table_add_view(lrm_table* t, const char* name, uint32_t source, const uint32_t* dims, int rank, uint64_t eoff,
                       uint32_t* token) {
    return guard([&] {
        need_ptr(t, "table");
        if (rank < 0 || (rank > 0 && !dims)) throw std::invalid_argument("bad dims");
        uint32_t tok = t->t.add_view(name ? name : "", source, std::vector<uint32_t>(dims, dims + rank), eoff);
        if (token) *token = tok;
    });
}

int lrm_table_seal(lrm_table* t, uint8_t* image) {
    return guard([&] {
        need_ptr(t, "table");
        t->t.seal();
        if (image) std::memcpy(image, t->t.image().data(), kTableBytes);
    });
}

void lrm_table_destroy(lrm_table* t) { delete t; }

int lrm_prepare(const uint8_t* image, const uint32_t* arenas, const uint64_t* bytes, int pages, uint32_t kernel,
                const uint32_t in[32], uint32_t out[32], int64_t grid[3], uint32_t physical[3]) {
    return guard([&] {
        need_ptr(image, "table image");
        need_ptr(in, "words");
        HeapLayout layout = layout_of(arenas, bytes, pages);
        (void)layout;
        PreparedDispatch pd = prepare(SealedTableView{image}, int(kernel), in);
        if (out) std::memcpy(out, pd.words.data(), 128);
        if (grid) {
            grid[0] = pd.grid.x;
            grid[1] = pd.grid.y;
            grid[2] = pd.grid.z;
        }
        if (physical) {
            physical[0] = pd.physical.x;
            physical[1] = pd.physical.y;
            physical[2] = pd.physical.z;
        }
    });
}

// ---------------------------------------------------------------- device

static void fill_info(const DeviceInfo& s, lrm_hip_device_info* o) {
    std::memset(o, 0, sizeof *o);
    o->index = s.index;
    copy_str(o->name, sizeof o->name, s.name);
    copy_str(o->arch, sizeof o->arch, s.arch);
    o->vendor_id = s.vendor_id;
    o->pci_device_id = s.pci_device_id;
    copy_str(o->pci_bus, sizeof o->pci_bus, s.pci_bus);
    copy_str(o->driver, sizeof o->driver, s.driver);
    o->memory_bytes = s.memory_bytes;
    o->compute_units = s.compute_units;
}

int lrm_hip_enumerate(lrm_hip_device_info* infos, int cap, int* count) {
    return guard([&] {
        auto all = Device::enumerate();
        if (count) *count = int(all.size());
        for (size_t i = 0; i < all.size() && int(i) < cap && infos; ++i) fill_info(all[i], &infos[i]);
    });
}

int lrm_hip_create(int index, uint32_t flags, lrm_hip_device** out) {
    return guard([&] {
        need_ptr(out, "out");
        *out = new lrm_hip_device(index, flags);
    });
}

int lrm_hip_destroy(lrm_hip_device* d) {
    return guard([&] { delete d; });
}

int lrm_hip_info(lrm_hip_device* d, lrm_hip_device_info* out) {
    return guard([&] {
        need_ptr(d, "device");
        need_ptr(out, "out");
        fill_info(d->d.info(), out);
    });
}

int lrm_hip_create_heap(lrm_hip_device* d, const uint32_t* arenas, const uint64_t* bytes, int pages) {
    return guard([&] {
        need_ptr(d, "device");
        d->d.create_heap(layout_of(arenas, bytes, pages));
    });
}

int lrm_hip_write_table(lrm_hip_device* d, const void* image, uint64_t bytes) {
    return guard([&] {
        need_ptr(d, "device");
        need_ptr(image, "image");
        d->d.write_table(image, bytes);
    });
}

int lrm_hip_upload(lrm_hip_device* d, int slot, uint64_t off, const void* src, uint64_t bytes) {
    return guard([&] {
        need_ptr(d, "device");
        need_ptr(src, "src");
        d->d.upload(slot, off, src, bytes);
    });
}

int lrm_hip_download(lrm_hip_device* d, int slot, uint64_t off, void* dst, uint64_t bytes) {
    return guard([&] {
        need_ptr(d, "device");
        need_ptr(dst, "dst");
        d->d.download(slot, off, dst, bytes);
    });
}

int lrm_hip_load_kernels(lrm_hip_device* d, uint8_t hash[32]) {
    return lrm_hip_load_kernel_set(d, LRM_HIP_KERNELS_REFERENCE, hash);
}

int lrm_hip_load_kernel_set(lrm_hip_device* d, uint32_t set, uint8_t hash[32]) {
    return guard([&] {
        need_ptr(d, "device");
        if (set != LRM_HIP_KERNELS_REFERENCE && set != LRM_HIP_KERNELS_FAST) contract_fail("unknown kernel set %u", set);
        auto h = d->d.load_kernels(set == LRM_HIP_KERNELS_FAST ? Device::KernelSet::Fast : Device::KernelSet::Reference);
        if (hash) std::memcpy(hash, h.data(), 32);
    });
}

int lrm_hip_debug_gemm_stamps(lrm_hip_device* d, uint32_t kind, uint64_t* dst, uint64_t words) {
    return guard([&] {
        need_ptr(d, "device");
        need_ptr(dst, "dst");
        hip_check(hipSetDevice(d->d.index()), "hipSetDevice");
        if (!gemm_stamps_read(int(kind), dst, size_t(words)))
            throw std::invalid_argument("no GEMM stamps: this library is not the stage-timing build, or kind " +
                                        std::to_string(kind) + " / " + std::to_string(words) + " words is out of range");
    });
}

int lrm_hip_contains(lrm_hip_device* d, uint32_t kernel) {
    if (!d) return 0;
    return d->d.kernels_loaded() && d->d.contains(int(kernel)) ? 1 : 0;
}

int lrm_hip_denormal_probe(lrm_hip_device* d, int* mode, uint32_t results[7]) {
    return guard([&] {
        need_ptr(d, "device");
        if (!d->d.kernels_loaded()) contract_fail("the denormal probe runs after LoadKernels");
        if (mode) *mode = d->d.denormal_mode();
        if (results) std::memcpy(results, d->d.denormal_results().data(), 28);
    });
}

int lrm_hip_begin(lrm_hip_device* d, int reusable, lrm_hip_list** out) {
    return guard([&] {
        need_ptr(d, "device");
        need_ptr(out, "out");
        *out = new lrm_hip_list{d->d.begin(reusable != 0), d};
    });
}

int lrm_hip_dispatch(lrm_hip_list* l, uint32_t kernel, const uint32_t words[32]) {
    return guard([&] {
        need_ptr(l, "list");
        need_ptr(words, "words");
        l->l->dispatch(int(kernel), words);
    });
}

int lrm_hip_dispatch_overlapped(lrm_hip_list* l, uint32_t kernel, const uint32_t words[32]) {
    return guard([&] {
        need_ptr(l, "list");
        need_ptr(words, "words");
        l->l->dispatch_overlapped(int(kernel), words);
    });
}

int lrm_hip_dispatch_decode_attention_static(lrm_hip_list* l, const uint32_t words[32], uint32_t y) {
    return guard([&] {
        need_ptr(l, "list");
        need_ptr(words, "words");
        record_decode_attention_static(l->owner->d, l->l, words, y);
    });
}

int lrm_hip_barrier(lrm_hip_list* l) {
    return guard([&] {
        need_ptr(l, "list");
        l->l->barrier();
    });
}

int lrm_hip_copy(lrm_hip_list* l, int ss, uint64_t so, int ds, uint64_t dof, uint64_t bytes) {
    return guard([&] {
        need_ptr(l, "list");
        l->l->copy(ss, so, ds, dof, bytes);
    });
}

int lrm_hip_begin_timer(lrm_hip_list* l, const char* name, int* timer) {
    return guard([&] {
        need_ptr(l, "list");
        int t = l->l->begin_timer(name ? name : "");
        if (timer) *timer = t;
    });
}

int lrm_hip_end_timer(lrm_hip_list* l, int timer) {
    return guard([&] {
        need_ptr(l, "list");
        l->l->end_timer(timer);
    });
}

int lrm_hip_submit(lrm_hip_device* d, lrm_hip_list* l, uint32_t repeat, uint64_t* fence) {
    return guard([&] {
        need_ptr(d, "device");
        need_ptr(l, "list");
        if (l->owner != d) contract_fail("the command list belongs to another backend");
        uint64_t f = d->d.submit(l->l, repeat);
        if (fence) *fence = f;
    });
}

int lrm_hip_wait(lrm_hip_device* d, uint64_t fence, int* dispatches, int* timers) {
    return guard([&] {
        need_ptr(d, "device");
        const Completion& c = d->d.wait(fence);
        if (dispatches) *dispatches = c.dispatches;
        if (timers) *timers = int(c.timers.size());
    });
}

int lrm_hip_timer(lrm_hip_device* d, uint64_t fence, int index, char* name, int cap, int64_t* start, int64_t* dur) {
    return guard([&] {
        need_ptr(d, "device");
        const Completion& c = d->d.wait(fence);
        if (index < 0 || index >= int(c.timers.size())) contract_fail("submission has no timer %d", index);
        const TimerResult& t = c.timers[size_t(index)];
        copy_str(name, cap, t.name.c_str());
        if (start) *start = t.start_ns;
        if (dur) *dur = t.duration_ns;
    });
}

int lrm_hip_release(lrm_hip_device* d, lrm_hip_list* l) {
    return guard([&] {
        need_ptr(d, "device");
        need_ptr(l, "list");
        d->d.release(l->l);
        delete l;
    });
}

// ---------------------------------------------------------------- executor

int lrm_qwen_create(lrm_hip_device* d, const lrm_qwen_config* c, const uint32_t* inv, int half, lrm_qwen** out) {
    return guard([&] {
        need_ptr(d, "device");
        need_ptr(c, "config");
        need_ptr(inv, "inv_freq_bits");
        need_ptr(out, "out");
        if (half * 2 != c->head_dim) throw std::invalid_argument("inv_freq_bits must hold head_dim / 2 words");
        QwenConfig qc{c->layers, c->hidden, c->heads, c->kv_heads, c->head_dim, c->intermediate, c->vocab, c->max_pos,
                      c->eps,    c->mode,   c->max_tokens, c->batch < 1 ? 1 : c->batch, c->taps};
        *out = new lrm_qwen(d, qc, inv);
    });
}

int lrm_qwen_destroy(lrm_qwen* q) {
    return guard([&] { delete q; });
}

int lrm_qwen_set_weight(lrm_qwen* q, const char* name, const uint16_t* data, uint64_t elems) {
    return guard([&] {
        need_ptr(q, "model");
        need_ptr(name, "name");
        need_ptr(data, "data");
        q->q.set_weight(name, data, elems);
    });
}

int lrm_qwen_read_weight(lrm_qwen* q, const char* name, uint16_t* out, uint64_t elems) {
    return guard([&] {
        need_ptr(q, "model");
        need_ptr(name, "name");
        need_ptr(out, "out");
        q->q.read_weight(name, out, elems);
    });
}

int lrm_qwen_forward(lrm_qwen* q, int seq, int pos0, const int32_t* ids, int t, float* logits, int rows, uint32_t* am) {
    return guard([&] {
        need_ptr(q, "model");
        need_ptr(ids, "ids");
        uint32_t a = q->q.forward(seq, pos0, ids, t, logits, logits ? rows : 0);
        if (am) *am = a;
    });
}

int lrm_qwen_greedy(lrm_qwen* q, const int32_t* prompt, int plen, int steps, int32_t* out) {
    return guard([&] {
        need_ptr(q, "model");
        need_ptr(prompt, "prompt");
        need_ptr(out, "out_ids");
        q->q.greedy(prompt, plen, steps, out);
    });
}

int lrm_qwen_decode_set(lrm_qwen* q, const int32_t* ids, const int32_t* pos) {
    return guard([&] {
        need_ptr(q, "model");
        need_ptr(ids, "ids");
        need_ptr(pos, "pos");
        q->q.set_decode_state(ids, pos);
    });
}

int lrm_qwen_decode_run(lrm_qwen* q, int steps) {
    return guard([&] {
        need_ptr(q, "model");
        q->q.run_decode_steps(steps);
    });
}

int lrm_qwen_decode_ids(lrm_qwen* q, int32_t* out, int count) {
    return guard([&] {
        need_ptr(q, "model");
        need_ptr(out, "out");
        q->q.read_decode_ids(out, count);
    });
}

int lrm_qwen_decode_batch(lrm_qwen* q, const int32_t* ids, const int32_t* pos, int steps, int32_t* out_ids) {
    return guard([&] {
        need_ptr(q, "model");
        need_ptr(ids, "ids");
        need_ptr(pos, "pos");
        need_ptr(out_ids, "out_ids");
        q->q.decode_batch(ids, pos, steps, out_ids);
    });
}

int lrm_qwen_read_logits(lrm_qwen* q, float* out, int rows) {
    return guard([&] {
        need_ptr(q, "model");
        need_ptr(out, "out");
        uint32_t tok = q->q.token("logits");
        TensorRow r = q->dev->d.table().row(tok);
        uint64_t bytes = uint64_t(rows) * uint64_t(q->q.config().vocab) * 4;
        if (rows < 0 || bytes > r.extent_bytes()) throw std::invalid_argument("logits rows out of range");
        q->dev->d.download(int(r.slot()), r.offset(), out, bytes);
    });
}

double lrm_qwen_last_ms(lrm_qwen* q) { return q ? q->q.last_ms() : -1.0; }

int lrm_qwen_persistent_decode(lrm_qwen* q) { return q ? (q->q.persistent_decode() ? 1 : 0) : -1; }

int lrm_qwen_swiglu_shift(lrm_qwen* q) { return q ? q->q.swiglu_shift() : -1; }

int lrm_qwen_set_swiglu_shift(lrm_qwen* q, int shift) {
    return guard([&] {
        need_ptr(q, "model");
        q->q.set_swiglu_shift_checked(shift);
    });
}

int lrm_qwen_token(lrm_qwen* q, const char* name, uint32_t* token) {
    return guard([&] {
        need_ptr(q, "model");
        need_ptr(name, "name");
        uint32_t t = q->q.token(name);
        if (token) *token = t;
    });
}

lrm_hip_device* lrm_qwen_device(lrm_qwen* q) { return q ? q->dev : nullptr; }

int lrm_qwen_tap_count(lrm_qwen* q) { return q ? q->q.tap_count() : 0; }

int lrm_qwen_tap_info(lrm_qwen* q, int i, char* name, int cap, int* width) {
    return guard([&] {
        need_ptr(q, "model");
        copy_str(name, cap, q->q.tap_name(i).c_str());
        if (width) *width = q->q.tap_width(i);
    });
}

int lrm_qwen_read_tap(lrm_qwen* q, int i, float* out, int rows) {
    return guard([&] {
        need_ptr(q, "model");
        need_ptr(out, "out");
        q->q.read_tap(i, out, rows);
    });
}

int lrm_qwen_read_cache(lrm_qwen* q, int seq, int layer, int which, int row0, int rows, float* out) {
    return guard([&] {
        need_ptr(q, "model");
        need_ptr(out, "out");
        q->q.read_cache(seq, layer, which, row0, rows, out);
    });
}

int lrm_qwen_write_cache(lrm_qwen* q, int seq, int layer, int which, int row0, int rows, const float* in) {
    return guard([&] {
        need_ptr(q, "model");
        need_ptr(in, "in");
        q->q.write_cache(seq, layer, which, row0, rows, in);
    });
}

int lrm_qwen_fill_cache_random(lrm_qwen* q, uint64_t seed, int rows) {
    return guard([&] {
        need_ptr(q, "model");
        q->q.fill_cache_random(seed, rows);
    });
}

// ---------------------------------------------------------------- inputs

uint64_t lrm_stream_of(const char* name) { return stream_of(name ? name : ""); }

int lrm_synth_normal_f32(uint64_t seed, uint64_t stream, uint64_t n, float std_, float* out) {
    return guard([&] {
        need_ptr(out, "out");
        synth_normal_f32(seed, stream, n, std_, out);
    });
}

int lrm_synth_normal_bf16(uint64_t seed, uint64_t stream, uint64_t n, float std_, uint16_t* out) {
    return guard([&] {
        need_ptr(out, "out");
        synth_normal_bf16(seed, stream, n, std_, out);
    });
}

int lrm_rope_table(const uint32_t* inv, int half, int max_pos, float* c, float* s) {
    return guard([&] {
        need_ptr(inv, "inv_freq_bits");
        need_ptr(c, "cos");
        need_ptr(s, "sin");
        rope_table(inv, half, max_pos, c, s);
    });
}

// ---------------------------------------------------------------- safetensors

struct lrm_st {
    std::unique_ptr<StFile> f;
};

static void copy_bytes(char* dst, int cap, int32_t* len, const std::string& s) {
    if (len) *len = int32_t(s.size());
    if (dst && cap > 0) std::memcpy(dst, s.data(), std::min(size_t(cap), s.size()));
}

int lrm_st_open(const char* path, lrm_st** out) {
    return guard([&] {
        need_ptr(path, "path");
        need_ptr(out, "out");
        *out = new lrm_st{StFile::open(path)};
    });
}

int lrm_st_open_verified(const char* path, int64_t bytes, const char* sha256_hex, lrm_st** out) {
    return guard([&] {
        need_ptr(path, "path");
        need_ptr(sha256_hex, "sha256");
        need_ptr(out, "out");
        std::string h(sha256_hex);
        for (char& ch : h) ch = char(std::tolower(uint8_t(ch)));
        if (h.size() != 64 || h.find_first_not_of("0123456789abcdef") != std::string::npos)
            throw std::invalid_argument("sha256 must be 64 hex digits");
        if (bytes < 0) throw std::invalid_argument("the pinned size is negative");
        *out = new lrm_st{StFile::open(path, bytes, h.c_str())};
    });
}

int lrm_st_validate(const uint8_t* bytes, uint64_t n, lrm_st** out) {
    return guard([&] {
        if (n) need_ptr(bytes, "bytes");
        need_ptr(out, "out");
        static const uint8_t none = 0;
        *out = new lrm_st{StFile::from_memory(n ? bytes : &none, n)};
    });
}

int lrm_st_info(const lrm_st* f, int64_t* header_length, int64_t* data_offset, int32_t* entries, int32_t* metadata,
                int32_t* aligned, uint64_t* length) {
    return guard([&] {
        need_ptr(f, "file");
        if (header_length) *header_length = f->f->header_length();
        if (data_offset) *data_offset = f->f->data_offset();
        if (entries) *entries = int32_t(f->f->entries().size());
        if (metadata) *metadata = int32_t(f->f->metadata().size());
        if (aligned) *aligned = f->f->aligned() ? 1 : 0;
        if (length) *length = f->f->length();
    });
}

int lrm_st_entry(const lrm_st* f, int i, char* name, int name_cap, int32_t* name_len, uint32_t* dtype, int32_t* rank,
                 int64_t* dims, int dims_cap, int64_t* begin, int64_t* end) {
    return guard([&] {
        need_ptr(f, "file");
        const auto& es = f->f->entries();
        if (i < 0 || size_t(i) >= es.size()) throw std::invalid_argument("entry " + std::to_string(i) + " of " + std::to_string(es.size()));
        const StEntry& e = es[size_t(i)];
        copy_bytes(name, name_cap, name_len, e.name);
        if (dtype) *dtype = e.dtype;
        if (rank) *rank = int32_t(e.shape.size());
        for (size_t k = 0; dims && k < e.shape.size() && int(k) < dims_cap; ++k) dims[k] = e.shape[k];
        if (begin) *begin = e.begin;
        if (end) *end = e.end;
    });
}

int lrm_st_metadata(const lrm_st* f, int i, char* key, int key_cap, int32_t* key_len, char* value, int value_cap,
                    int32_t* value_len) {
    return guard([&] {
        need_ptr(f, "file");
        const auto& m = f->f->metadata();
        if (i < 0 || size_t(i) >= m.size()) throw std::invalid_argument("metadata " + std::to_string(i) + " of " + std::to_string(m.size()));
        copy_bytes(key, key_cap, key_len, m[size_t(i)].first);
        copy_bytes(value, value_cap, value_len, m[size_t(i)].second);
    });
}

int lrm_st_data(const lrm_st* f, int i, const void** data) {
    return guard([&] {
        need_ptr(f, "file");
        need_ptr(data, "data");
        const auto& es = f->f->entries();
        if (i == -1) {
            *data = f->f->bytes();
            return;
        }
        if (i < 0 || size_t(i) >= es.size()) throw std::invalid_argument("entry " + std::to_string(i));
        *data = f->f->data(es[size_t(i)]);
    });
}

int lrm_st_close(lrm_st* f) {
    return guard([&] { delete f; });
}

int lrm_qwen_load_safetensors(lrm_qwen* q, const char* path) {
    return guard([&] {
        need_ptr(q, "model");
        need_ptr(path, "path");
        q->q.load_safetensors(path);
    });
}

// ---------------------------------------------------------------- tokenizer

struct lrm_tok {
    std::unique_ptr<tok::Tokenizer> t;
};

int lrm_tok_parse(const uint8_t* json, uint64_t n, lrm_tok** out) {
    return guard([&] {
        if (n) need_ptr(json, "json");
        need_ptr(out, "out");
        *out = new lrm_tok{tok::Tokenizer::parse(json, n)};
    });
}

int lrm_tok_destroy(lrm_tok* t) {
    return guard([&] { delete t; });
}

int lrm_tok_info(const lrm_tok* t, int32_t* vocab_size, int32_t* merges, int32_t* added) {
    return guard([&] {
        need_ptr(t, "tokenizer");
        if (vocab_size) *vocab_size = t->t->vocab_size();
        if (merges) *merges = t->t->merge_count();
        if (added) *added = int32_t(t->t->added().size());
    });
}

int lrm_tok_added(const lrm_tok* t, int i, int32_t* id, char* content, int cap, int32_t* len, int32_t* special) {
    return guard([&] {
        need_ptr(t, "tokenizer");
        const auto& a = t->t->added();
        if (i < 0 || size_t(i) >= a.size()) throw std::invalid_argument("added token " + std::to_string(i));
        if (id) *id = a[size_t(i)].id;
        if (special) *special = a[size_t(i)].special ? 1 : 0;
        copy_bytes(content, cap, len, tok::utf8_encode(a[size_t(i)].content));
    });
}

int lrm_tok_encode(const lrm_tok* t, const uint8_t* utf8, uint64_t n, int32_t* ids, uint64_t cap, uint64_t* count) {
    return guard([&] {
        need_ptr(t, "tokenizer");
        if (n) need_ptr(utf8, "text");
        const std::vector<int32_t> v = t->t->encode(utf8, n);
        fill_out(v.data(), v.size(), ids, cap, count);
    });
}

int lrm_tok_encode_bytes(const lrm_tok* t, const uint8_t* bytes, uint64_t n, int32_t* ids, uint64_t cap,
                         uint64_t* count) {
    return guard([&] {
        need_ptr(t, "tokenizer");
        if (n) need_ptr(bytes, "bytes");
        const std::vector<int32_t> v = t->t->encode_bytes(bytes, n);
        fill_out(v.data(), v.size(), ids, cap, count);
    });
}

int lrm_tok_decode_bytes(const lrm_tok* t, const int32_t* ids, uint64_t n, uint8_t* out, uint64_t cap,
                         uint64_t* len) {
    return guard([&] {
        need_ptr(t, "tokenizer");
        if (n) need_ptr(ids, "ids");
        const std::string b = t->t->decode_bytes(ids, n);
        fill_out(reinterpret_cast<const uint8_t*>(b.data()), b.size(), out, cap, len);
    });
}

int lrm_tok_id_of(const lrm_tok* t, const uint8_t* token, uint64_t n, int32_t* id) {
    return guard([&] {
        need_ptr(t, "tokenizer");
        need_ptr(id, "id");
        *id = t->t->id_of(std::string(reinterpret_cast<const char*>(token), n));
    });
}

int lrm_tok_token_of(const lrm_tok* t, int32_t id, char* out, int cap, int32_t* len) {
    return guard([&] {
        need_ptr(t, "tokenizer");
        need_ptr(len, "len");
        std::string s;
        if (!t->t->token_of(id, s)) {
            *len = -1;
            return;
        }
        copy_bytes(out, cap, len, s);
    });
}

int lrm_tok_pre_split(const uint8_t* utf8, uint64_t n, uint64_t* bounds, uint64_t cap, uint64_t* count) {
    return guard([&] {
        if (n) need_ptr(utf8, "text");
        std::u32string s;
        size_t bad = 0;
        if (!tok::utf8_decode(utf8, n, s, &bad)) throw std::invalid_argument("not valid UTF-8 at byte " + std::to_string(bad));
        const std::vector<size_t> b = tok::pre_split(s);
        // scalar boundaries -> byte offsets
        std::vector<uint64_t> off;
        off.reserve(b.size());
        uint64_t at = 0;
        size_t k = 0;
        for (size_t i = 0; i <= s.size(); ++i) {
            while (k < b.size() && b[k] == i) {
                off.push_back(at);
                ++k;
            }
            if (i < s.size()) {
                const uint32_t c = uint32_t(s[i]);
                at += c < 0x80 ? 1 : c < 0x800 ? 2 : c < 0x10000 ? 3 : 4;
            }
        }
        fill_out(off.data(), off.size(), bounds, cap, count);
    });
}

int lrm_tok_nfc(const uint8_t* utf8, uint64_t n, uint8_t* out, uint64_t cap, uint64_t* len) {
    return guard([&] {
        if (n) need_ptr(utf8, "text");
        std::u32string s;
        size_t bad = 0;
        if (!tok::utf8_decode(utf8, n, s, &bad)) throw std::invalid_argument("not valid UTF-8 at byte " + std::to_string(bad));
        const std::string r = tok::utf8_encode(tok::nfc(s));
        fill_out(reinterpret_cast<const uint8_t*>(r.data()), r.size(), out, cap, len);
    });
}

int lrm_tok_nfc_many(const uint8_t* text, const uint64_t* offsets, uint64_t count, uint8_t* out, uint64_t cap,
                     uint64_t* out_offsets, uint64_t* len) {
    return guard([&] {
        need_ptr(offsets, "offsets");
        need_ptr(len, "len");
        std::string all;
        std::vector<uint64_t> offs{0};
        for (uint64_t i = 0; i < count; ++i) {
            const uint64_t b = offsets[i], e = offsets[i + 1];
            if (e < b) throw std::invalid_argument("offsets decrease at " + std::to_string(i));
            std::u32string s;
            size_t bad = 0;
            if (!tok::utf8_decode(text + b, size_t(e - b), s, &bad))
                throw std::invalid_argument("string " + std::to_string(i) + " is not valid UTF-8");
            all += tok::utf8_encode(tok::nfc(s));
            offs.push_back(all.size());
        }
        *len = all.size();
        if (out && cap >= all.size()) {
            if (!all.empty()) std::memcpy(out, all.data(), all.size());
            if (out_offsets) std::memcpy(out_offsets, offs.data(), offs.size() * sizeof(uint64_t));
        }
    });
}

int lrm_tok_scalar_tables(uint8_t* classes, uint8_t* contraction, uint8_t* nfc_split) {
    return guard([&] {
        for (uint32_t c = 0; c < 0x110000; ++c) {
            if (classes) classes[c] = uint8_t(tok::char_class(c));
            if (contraction) contraction[c] = uint8_t(tok::contraction_letter(c));
            if (nfc_split) nfc_split[c] = tok::nfc_split_point(c) ? 1 : 0;
        }
    });
}

int lrm_tok_byte_char(int b, uint32_t* c) {
    return guard([&] {
        need_ptr(c, "c");
        if (b < 0 || b > 255) throw std::invalid_argument("byte " + std::to_string(b));
        *c = tok::byte_char(uint8_t(b));
    });
}

}  // extern "C"
