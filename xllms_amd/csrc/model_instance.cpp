// Model and model-instance entry points of the plugin: the decode path
// behind the reference scheduler's instance_exec call
// (src/core/scheduler.c:477-488), with the sequences' pages managed by the
// KV-cache index (kv_index.cpp) and the K/V caches resident in HBM.
// Declared, with the conventions, in include/xllm_hip_backend.h.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "batch_tables.h"
#include "paged_kv_append.h"
#include "paged_decode_rows.h"
#include "workspace.h"
#include "xllm_hip_backend.h"
#include "xllm_hip_kv_index.h"

#define XMI_EXPORT extern "C" __attribute__((visibility("default")))

namespace {

constexpr uint32_t kModelMagic = 0x584d444cu;  // "XMDL"
constexpr uint32_t kInstMagic = 0x58494e53u;   // "XINS"
constexpr int kDefaultMaxBatch = 256;

struct ModelSpec {
    uint32_t magic = kModelMagic;
    int num_blocks = 0, num_kv_heads = 0, block_size = 0, head_size = 0, num_heads = 0;
    int kv_dtype = 0, elem_bytes = 0, max_batch = 0, max_blocks = 0;
    float scale = 0.f;
};

int fail(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
int fail(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::fprintf(stderr, "[hip_backend] ");
    std::vfprintf(stderr, fmt, ap);
    std::fprintf(stderr, "\n");
    va_end(ap);
    return -1;
}

// Grow-only device / pinned host buffers, reused across execs (an exec
// waits for its device work before returning, so reuse is safe).
template <class T>
struct DevBuf {
    T *p = nullptr;
    size_t cap = 0;
    bool reserve(size_t n) {
        if (n <= cap) return true;
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
        if (hipMalloc((void **)&p, n * sizeof(T)) != hipSuccess) return false;
        cap = n;
        return true;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
    }
};

template <class T>
struct HostBuf {
    T *p = nullptr;
    size_t cap = 0, n = 0;
    bool reserve(size_t want) {
        if (want <= cap) return true;
        size_t c = cap ? cap : 256;
        while (c < want) c *= 2;
        T *q = nullptr;
        if (hipHostMalloc((void **)&q, c * sizeof(T), hipHostMallocDefault) != hipSuccess)
            return false;
        if (p) {
            std::memcpy(q, p, n * sizeof(T));
            (void)hipHostFree(p);
        }
        p = q;
        cap = c;
        return true;
    }
    bool push(const T &v) {
        if (!reserve(n + 1)) return false;
        p[n++] = v;
        return true;
    }
    void release() {
        if (p) (void)hipHostFree(p);
        p = nullptr;
        cap = n = 0;
    }
};

struct InstanceState {
    uint32_t magic = kInstMagic;
    ModelSpec spec;
    int device = 0;
    hipStream_t stream = nullptr;
    void *key_cache = nullptr;
    void *value_cache = nullptr;
    NxtKvIndex *index = nullptr;
    std::unordered_map<std::string, int32_t> seqs;  // request id -> sequence
    struct Bound {
        NxtDecodeIo io;               // token_ids points into `tokens`
        uint64_t exec_stamp;          // the exec that last took it (duplicate check)
        std::vector<int32_t> tokens;  // the bound token ids (copied at bind)
        bool queued = false;          // deferred mode: in `pending`
    };
    std::unordered_map<std::string, Bound> bound;  // request id -> next exec's buffers
    uint64_t exec_stamp = 0;
    // deferred mode: requests queued by exec (their bound entries marked
    // queued), run as one batch at the flush
    bool deferred = false;
    std::vector<std::string> pending;
    std::vector<std::string> flushing;  // the batch being run (capacity kept)
    // staging of one exec
    HostBuf<int32_t> h_slots, h_src, h_dst, h_bt, h_lens, h_group, h_pblocks, h_seqs;
    HostBuf<const char *> h_kptr, h_vptr, h_qptr;
    HostBuf<char *> h_optr;
    HostBuf<char> h_pack;  // every array an exec uploads, 256-byte aligned parts
    DevBuf<char> d_pack;
    // completion word of the execs (host-coherent pinned memory; see
    // wait_exec) and the number the last exec's signal stored
    unsigned *done = nullptr;
    unsigned done_seq = 0;
    // One-request decode steps (fast_step): each sequence's length and block
    // table kept on the device between execs, in a record of rec_ints ints
    // per sequence handle ([0] the length, the table from kRecHead on), and
    // the number of tokens the record holds (-1: none), on the host.
    static constexpr int kRecHead = 4;
    // a record holds at most this many table entries (a model whose table
    // width is the whole pool would otherwise make every record that wide);
    // longer sequences take the general exec
    static constexpr int kRecMaxBlocks = 4096;
    int rec_blocks = 0;
    DevBuf<int32_t> d_recs;
    std::vector<int32_t> dev_len;
    size_t rec_ints = 0;
    DevBuf<float> d_state;      // fp32 rows [num_heads][head_size], then their lse [num_heads]
    HostBuf<int32_t> h_rec;     // staging of one record
    // The general exec's block tables, kept on the device between execs
    // (bt_dev, rows of bt.stride entries; bt: what they hold, and when an
    // exec may update them in place, batch_tables.h), the (index, page)
    // pairs of one exec's update (h_upd), and the batch's lengths before its
    // appends (h_len0).
    xhip::ResidentTables bt;
    DevBuf<int32_t> bt_dev;
    HostBuf<int32_t> h_upd, h_len0;

    void forget_device_row(int32_t seq) {
        if (seq >= 0 && (size_t)seq < dev_len.size()) dev_len[(size_t)seq] = -1;
        bt.forget(seq);  // (an admission that reuses the handle, a release or a failure)
    }
    // Records for handles [0, n): grown by doubling; a new buffer holds
    // none (the old records are dropped with it).
    bool ensure_recs(int32_t n) {
        if ((size_t)n <= dev_len.size()) return true;
        size_t cap = dev_len.empty() ? 64 : dev_len.size();
        while (cap < (size_t)n) cap *= 2;
        d_recs.release();
        if (!d_recs.reserve(cap * rec_ints)) {
            dev_len.clear();
            return false;
        }
        dev_len.assign(cap, -1);
        return true;
    }

    // Appends h's contents to h_pack at a 256-byte boundary; returns its
    // offset (h_pack.n becomes -1 when host memory runs out).
    template <class T>
    size_t pack(const HostBuf<T> &h) {
        if (h_pack.n == (size_t)-1) return 0;
        const size_t off = (h_pack.n + 255) & ~(size_t)255;
        const size_t bytes = h.n * sizeof(T);
        if (!h_pack.reserve(off + bytes)) {
            h_pack.n = (size_t)-1;
            return 0;
        }
        if (bytes) std::memcpy(h_pack.p + off, h.p, bytes);
        h_pack.n = bytes ? off + bytes : h_pack.n;
        return off;
    }
};

const NxtTensor *find_input(const NxtModelConfig &c, const char *name) {
    for (uint32_t i = 0; i < c.input_count; ++i)
        if (c.inputs && c.inputs[i] && c.inputs[i]->name && !std::strcmp(c.inputs[i]->name, name))
            return c.inputs[i];
    return nullptr;
}

bool is_device(const void *ptr) {
    hipPointerAttribute_t a;
    std::memset(&a, 0, sizeof(a));
    if (hipPointerGetAttributes(&a, ptr) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return a.type == hipMemoryTypeDevice || a.type == hipMemoryTypeManaged;
}

InstanceState *state_of(NxtModelInstance *inst) {
    if (!inst || !inst->instance_state) return nullptr;
    auto *st = (InstanceState *)inst->instance_state;
    return st->magic == kInstMagic ? st : nullptr;
}

int parse_spec(const NxtModel *m, ModelSpec &s) {
    const NxtTensor *kc = find_input(m->config, "key_cache");
    const NxtTensor *q = find_input(m->config, "query");
    if (!kc || !q || kc->dims_count != 4 || q->dims_count != 2 || !kc->shape || !q->shape)
        return fail("model %s: needs inputs \"key_cache\" [blocks, kv_heads, block_size, "
                    "head_size] and \"query\" [heads, head_size]",
                    m->name ? m->name : "?");
    s.num_blocks = (int)kc->shape[0];
    s.num_kv_heads = (int)kc->shape[1];
    s.block_size = (int)kc->shape[2];
    s.head_size = (int)kc->shape[3];
    s.num_heads = (int)q->shape[0];
    if (q->shape[1] != kc->shape[3])
        return fail("model: query head_size %lld != key_cache head_size %lld",
                    (long long)q->shape[1], (long long)kc->shape[3]);
    switch ((int)kc->dtype) {
        case NXT_TYPE_FP16: s.kv_dtype = NXT_KV_FP16; s.elem_bytes = 2; break;
        case NXT_TYPE_FP32: s.kv_dtype = NXT_KV_FP32; s.elem_bytes = 4; break;
        case NXT_TYPE_BF16_HIP: s.kv_dtype = NXT_KV_BF16; s.elem_bytes = 2; break;
        default: return fail("model: key_cache dtype %d is not FP16, FP32 or BF16", kc->dtype);
    }
    s.max_batch = m->config.max_batch_size > 0 ? m->config.max_batch_size : kDefaultMaxBatch;
    const NxtTensor *bt = find_input(m->config, "block_tables");
    s.max_blocks = (bt && bt->dims_count == 2 && bt->shape && bt->shape[1] > 0)
                       ? (int)bt->shape[1]
                       : s.num_blocks;
    const long long bound = (1LL << 28) / std::max(1, s.block_size);
    if (s.max_blocks > bound) s.max_blocks = (int)bound;
    if (s.num_blocks <= 0 || s.num_kv_heads <= 0 || s.num_heads <= 0 ||
        s.num_heads % s.num_kv_heads || s.head_size <= 0 || (s.head_size * s.elem_bytes) % 16 ||
        s.block_size <= 0 || (s.block_size & (s.block_size - 1)))
        return fail("model: unsupported geometry (blocks %d, kv heads %d, heads %d, head_size "
                    "%d, block_size %d)",
                    s.num_blocks, s.num_kv_heads, s.num_heads, s.head_size, s.block_size);
    s.scale = 1.0f / std::sqrt((float)s.head_size);
    return 0;
}

void destroy_state(InstanceState *st) {
    if (!st) return;
    if (st->stream) (void)hipStreamSynchronize(st->stream);
    if (st->index) nxt_kv_index_destroy(st->index);
    if (st->key_cache) (void)hipFree(st->key_cache);
    if (st->value_cache) (void)hipFree(st->value_cache);
    for (auto *b : {&st->h_slots, &st->h_src, &st->h_dst, &st->h_bt, &st->h_lens, &st->h_group,
                    &st->h_pblocks, &st->h_seqs})
        b->release();
    st->h_kptr.release();
    st->h_vptr.release();
    st->h_qptr.release();
    st->h_optr.release();
    st->h_pack.release();
    st->d_pack.release();
    st->d_recs.release();
    st->d_state.release();
    st->h_rec.release();
    st->bt_dev.release();
    st->h_upd.release();
    st->h_len0.release();
    if (st->done) (void)hipHostFree(st->done);
    st->done = nullptr;
    // the operator layer keeps split-K / cascade workspaces per stream:
    // free this stream's before the handle goes (it may be reused)
    if (st->stream) (void)xhip_release_stream_workspaces(st->device, st->stream);
    if (st->stream) (void)hipStreamDestroy(st->stream);
    st->magic = 0;
    delete st;
}

// With XLLM_HIP_EXEC_TRACE=1 in the environment, each exec prints the host
// time of its phases (microseconds) to stderr.
struct PhaseTrace {
    using clock = std::chrono::steady_clock;
    explicit PhaseTrace(clock::time_point t0) : last(t0), on(enabled()) {}
    static bool enabled() {
        static const bool e = [] {
            const char *v = std::getenv("XLLM_HIP_EXEC_TRACE");
            return v && *v && *v != '0';
        }();
        return e;
    }
    void mark(const char *name) {
        if (!on || n >= 8) return;
        const clock::time_point t = clock::now();
        names[n] = name;
        us[n++] = std::chrono::duration<double, std::micro>(t - last).count();
        last = t;
    }
    void report(uint32_t requests) const {
        if (!on) return;
        std::fprintf(stderr, "[hip_backend] exec %u requests:", requests);
        for (int i = 0; i < n; ++i) std::fprintf(stderr, " %s %.1f", names[i], us[i]);
        std::fprintf(stderr, " us\n");
    }
    clock::time_point last;
    bool on;
    int n = 0;
    const char *names[8];
    double us[8];
};

// XLLM_HIP_EXEC_SYNC=1 (read once): execs wait with hipStreamSynchronize
// instead of the completion word.  A diagnostic switch, for comparing the two.
bool exec_sync_forced() {
    static const bool forced = [] {
        const char *v = std::getenv("XLLM_HIP_EXEC_SYNC");
        return v && v[0] == '1';
    }();
    return forced;
}

// Waits until the device has run everything this exec queued on the
// instance's stream.  A one-thread kernel queued last stores the exec's
// number to the host-coherent completion word (it starts only once the
// exec's kernels have finished), and the host polls the word: measured on
// MI355X the host sees it ~2 us before hipStreamSynchronize returns.  If the
// signal cannot be queued, or the word has not changed after 2 ms (long
// work, or a kernel that failed, after which the queue runs nothing more),
// hipStreamSynchronize waits instead and reports the stream's error.
hipError_t wait_exec(InstanceState *st) {
    if (!st->done || exec_sync_forced()) return hipStreamSynchronize(st->stream);
    unsigned v = st->done_seq + 1;
    if (v == 0) v = 1;  // (the word starts at 0)
    if (xhip::launch_exec_signal(st->done, v, st->stream) != hipSuccess) {
        (void)hipGetLastError();
        return hipStreamSynchronize(st->stream);
    }
    st->done_seq = v;
    using clock = std::chrono::steady_clock;
    const clock::time_point t0 = clock::now();
    while (__atomic_load_n(st->done, __ATOMIC_ACQUIRE) != v) {
#if defined(__x86_64__)
        __builtin_ia32_pause();
#endif
        if (clock::now() - t0 > std::chrono::milliseconds(2)) return hipStreamSynchronize(st->stream);
    }
    return hipSuccess;
}

struct Item {
    std::string id;
    NxtDecodeIo io;
    int32_t seq;  // -1: admitted by this exec
    // (general exec) the sequence's length before this exec's tokens (-1:
    // admitted by it), and its pages opened by them: entries [open0, open0 +
    // nopen) of the exec's (table entry, page) list
    int32_t len0 = -1;
    size_t open0 = 0, nopen = 0;
};

int exec_ids(NxtModelInstance *instance, InstanceState *st, const std::vector<std::string> &ids);

// Runs the queued requests of deferred mode as one exec.
int flush_pending(NxtModelInstance *instance, InstanceState *st) {
    if (st->pending.empty()) return 0;
    st->flushing.swap(st->pending);
    st->pending.clear();
    for (const std::string &id : st->flushing) {
        auto b = st->bound.find(id);
        if (b != st->bound.end()) b->second.queued = false;
    }
    const int rc = exec_ids(instance, st, st->flushing);
    st->flushing.clear();
    return rc;
}

}  // namespace

XMI_EXPORT int nxt_model_init(NxtModel *model) {
    if (!model) return -1;
    ModelSpec spec;
    if (parse_spec(model, spec) != 0) return -1;
    auto *ms = new (std::nothrow) ModelSpec(spec);
    auto *inst = (NxtModelInstance *)std::calloc(1, sizeof(NxtModelInstance));
    if (!ms || !inst) {
        delete ms;
        std::free(inst);
        return -1;
    }
    model->backend_state = ms;
    inst->model = model;
    const std::string name = std::string(model->name ? model->name : "model") + "_0";
    inst->name = strdup(name.c_str());
    inst->kind = NXT_INSTANCE_KIND_GPU;
    if (hipGetDevice(&inst->device_id) != hipSuccess || nxt_model_instance_init(inst) != 0) {
        std::free(inst->name);
        std::free(inst);
        delete ms;
        model->backend_state = nullptr;
        return -1;
    }
    model->instances = inst;
    model->instance_count = 1;
    return 0;
}

XMI_EXPORT int nxt_model_fini(NxtModel *model) {
    if (!model) return -1;
    for (uint32_t i = 0; model->instances && i < model->instance_count; ++i) {
        nxt_model_instance_fini(&model->instances[i]);
        std::free(model->instances[i].name);
    }
    std::free(model->instances);
    model->instances = nullptr;
    model->instance_count = 0;
    auto *ms = (ModelSpec *)model->backend_state;
    if (ms && ms->magic == kModelMagic) delete ms;
    model->backend_state = nullptr;
    return 0;
}

XMI_EXPORT int nxt_model_instance_init(NxtModelInstance *instance) {
    if (!instance || !instance->model || !instance->model->backend_state) return -1;
    const auto *ms = (const ModelSpec *)instance->model->backend_state;
    if (ms->magic != kModelMagic) return -1;
    auto *st = new (std::nothrow) InstanceState;
    if (!st) return -1;
    st->spec = *ms;
    st->device = instance->device_id;
    const ModelSpec &s = st->spec;
    const size_t cache_bytes = (size_t)s.num_blocks * s.num_kv_heads * s.block_size *
                               s.head_size * s.elem_bytes;
    hipError_t e = hipSetDevice(st->device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&st->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipMalloc(&st->key_cache, cache_bytes);
    if (e == hipSuccess) e = hipMalloc(&st->value_cache, cache_bytes);
    if (e == hipSuccess) e = hipHostMalloc((void **)&st->done, 64, hipHostMallocCoherent);
    if (e == hipSuccess) *st->done = 0;
    if (e == hipSuccess && !st->d_state.reserve((size_t)s.num_heads * (s.head_size + 1)))
        e = hipErrorOutOfMemory;
    // a record: the head, then a table row, in whole 256-byte units
    st->rec_blocks = std::min(s.max_blocks, InstanceState::kRecMaxBlocks);
    st->rec_ints = ((size_t)InstanceState::kRecHead + (size_t)st->rec_blocks + 63) & ~(size_t)63;
    if (e != hipSuccess) {
        destroy_state(st);
        return fail("instance init: %s (K/V caches of %zu bytes each)", hipGetErrorString(e),
                    cache_bytes);
    }
    st->index = nxt_kv_index_create(s.num_blocks, s.block_size, s.max_blocks);
    if (!st->index) {
        destroy_state(st);
        return fail("instance init: out of memory");
    }
    instance->instance_state = st;
    instance->exec_count = 0;
    instance->total_exec_ms = 0.0;
    return 0;
}

XMI_EXPORT int nxt_model_instance_fini(NxtModelInstance *instance) {
    if (!instance) return -1;
    InstanceState *st = state_of(instance);
    if (st) (void)flush_pending(instance, st);  // queued requests still run
    destroy_state(st);
    instance->instance_state = nullptr;
    return 0;
}

XMI_EXPORT int nxt_model_instance_bind(NxtModelInstance *instance, const char *request_id,
                                       const NxtDecodeIo *io) {
    InstanceState *st = state_of(instance);
    if (!st || !request_id || !io) return -1;
    if (io->struct_size < sizeof(NxtDecodeIo)) return fail("bind: struct_size %u", io->struct_size);
    if (io->num_tokens < 0) return fail("bind: num_tokens %d", io->num_tokens);
    if (io->num_tokens > 0 && (!io->token_ids || !io->key || !io->value))
        return fail("bind %s: tokens without token_ids / key / value", request_id);
    if (!io->query != !io->output) return fail("bind %s: query and output go together", request_id);
    for (const void *p : {io->key, io->value, io->query, (const void *)io->output}) {
        if (!p) continue;
        if (((uintptr_t)p & 15) || !is_device(p))
            return fail("bind %s: buffers must be 16-byte aligned device memory", request_id);
    }
    if (st->deferred) {
        auto q = st->bound.find(request_id);
        if (q != st->bound.end() && q->second.queued) {
            // its queued exec consumes the current binding first
            const int rc = flush_pending(instance, st);
            if (rc != 0) return rc;
        }
    }
    InstanceState::Bound &b = st->bound[request_id];
    b.tokens.assign(io->token_ids, io->token_ids + io->num_tokens);
    b.io = *io;
    b.io.struct_size = sizeof(NxtDecodeIo);
    b.io.token_ids = b.tokens.empty() ? nullptr : b.tokens.data();
    b.exec_stamp = 0;
    b.queued = false;
    return 0;
}

XMI_EXPORT int nxt_model_instance_exec(NxtModelInstance *instance, NxtInferRequest **requests,
                                       uint32_t request_count) {
    InstanceState *st = state_of(instance);
    if (!st || (request_count && !requests)) return -1;
    for (uint32_t i = 0; i < request_count; ++i)
        if (!requests[i] || !requests[i]->request_id) return fail("exec: request %u has no id", i);
    if (!st->deferred) {
        std::vector<std::string> ids;
        ids.reserve(request_count);
        for (uint32_t i = 0; i < request_count; ++i) ids.emplace_back(requests[i]->request_id);
        return exec_ids(instance, st, ids);
    }
    if (request_count == 0) return flush_pending(instance, st);
    for (uint32_t i = 0; i < request_count; ++i) {
        const char *id = requests[i]->request_id;
        auto b = st->bound.find(id);
        if (b != st->bound.end() && b->second.queued) {
            // its next step: run the queued batch first (which consumes the
            // binding, so this exec then finds none)
            const int rc = flush_pending(instance, st);
            if (rc != 0) return rc;
            b = st->bound.find(id);
        }
        if (b == st->bound.end()) return fail("exec: request %s has no bound buffers", id);
        b->second.queued = true;
        st->pending.emplace_back(id);
        if ((int)st->pending.size() >= st->spec.max_batch) {
            const int rc = flush_pending(instance, st);
            if (rc != 0) return rc;
        }
    }
    return 0;
}

XMI_EXPORT int nxt_model_instance_flush(NxtModelInstance *instance) {
    InstanceState *st = state_of(instance);
    if (!st) return -1;
    return flush_pending(instance, st);
}

XMI_EXPORT int nxt_model_instance_set_deferred(NxtModelInstance *instance, int on) {
    InstanceState *st = state_of(instance);
    if (!st) return -1;
    if (on) {
        st->deferred = true;
        return 0;
    }
    st->deferred = false;
    return flush_pending(instance, st);
}

namespace {

// One-request decode steps -- the reference scheduler's instance_exec(.., 1)
// for a running request: one token appended, a query to attend with, a head
// size the new-token fold supports.
bool fast_ok(const InstanceState *st, const std::vector<Item> &items) {
    if (items.size() != 1) return false;
    const Item &it = items[0];
    const int d = st->spec.head_size;
    if (it.seq < 0 || it.io.num_tokens != 1 || !it.io.query || !it.io.output || !st->d_state.p ||
        !(d == 32 || d == 64 || d == 128))
        return false;
    // the sequence with its new token fits a record
    const long long len = (long long)nxt_kv_seq_len(st->index, it.seq) + 1;
    return len <= (long long)st->rec_blocks * st->spec.block_size;
}

// A one-request decode step without the staging launch: the sequence's
// length and block table are already on the device (its record, uploaded
// by one staging copy when it does not hold exactly the tokens before this
// one), the attention runs over those cached tokens, and its merge folds in
// the new token from the request's bound rows and then stores them to the
// token's cache slot, the new page id to the record when the token opens a
// page, and the new length (xhip_paged_attention_fold_new).
int fast_step(InstanceState *st, Item &it) {
    const ModelSpec &s = st->spec;
    const int L = nxt_kv_seq_len(st->index, it.seq) + 1;  // with the new token
    const int width = (L + s.block_size - 1) / s.block_size;
    const size_t n = ((size_t)InstanceState::kRecHead + (size_t)width + 3) & ~(size_t)3;
    // (what can run out, before the index takes the token: after that its
    // rows must reach the cache)
    if (!st->ensure_recs(it.seq + 1)) return fail("exec: out of device memory");
    if (!st->h_rec.reserve(n)) return fail("exec: out of host memory");
    int32_t slot = -1;
    const int r = nxt_kv_seq_append(st->index, it.seq, it.io.token_ids, 1, &slot);
    if (r != NXT_KV_OK) return fail("exec: appending to %s failed (%d)", it.id.c_str(), r);
    int32_t *rec = st->d_recs.p + (size_t)it.seq * st->rec_ints;
    if (st->dev_len[(size_t)it.seq] != L - 1) {
        st->dev_len[(size_t)it.seq] = -1;
        std::memset(st->h_rec.p, 0, n * sizeof(int32_t));
        int32_t len_now = 0;
        if (nxt_kv_batch_tables(st->index, &it.seq, 1, width,
                                st->h_rec.p + InstanceState::kRecHead, &len_now) != NXT_KV_OK ||
            len_now != L)
            return fail("exec: block table of %s", it.id.c_str());
        st->h_rec.p[0] = L - 1;
        const hipError_t e = xhip::launch_stage_copy(rec, st->h_rec.p, n * sizeof(int32_t),
                                                     st->stream);
        if (e != hipSuccess) return fail("exec: record upload: %s", hipGetErrorString(e));
    }
    const int last = L - 1;  // the new token's position
    int *entry = last % s.block_size == 0
                     ? rec + InstanceState::kRecHead + last / s.block_size
                     : nullptr;
    const int kbs = s.num_kv_heads * s.block_size * s.head_size;
    const int khs = s.block_size * s.head_size;
    const int a = xhip_paged_attention_fold_new(
        it.io.output, it.io.query, st->key_cache, st->value_cache,
        rec + InstanceState::kRecHead, rec, st->d_state.p,
        st->d_state.p + (size_t)s.num_heads * s.head_size, it.io.key, it.io.value, entry, rec,
        slot, slot / s.block_size, L, s.num_heads, s.head_size, s.num_kv_heads, s.scale, width,
        s.block_size, kbs, khs, s.kv_dtype, st->stream);
    if (a != NXT_ATTN_OK) return fail("exec: attention: %s", nxt_attn_last_error());
    st->dev_len[(size_t)it.seq] = L;
    return 0;
}

// The general exec (admissions, appends, any batch): index work on the host,
// one staging launch for every array the launches read (with the new rows'
// K/V write), the copies of partly shared pages and the attention.
int slow_step(InstanceState *st, std::vector<Item> &items, PhaseTrace &tr) {
    const ModelSpec &s = st->spec;
    // 1. sequences: admissions and appends; the K/V rows to write and copy
    const size_t kv_row = (size_t)s.num_kv_heads * s.head_size * s.elem_bytes;
    st->h_slots.n = st->h_src.n = st->h_dst.n = st->h_kptr.n = st->h_vptr.n = 0;
    std::vector<int32_t> mapping, src, dst, slots;
    std::vector<std::pair<int32_t, int32_t>> opened;  // (table entry, page) of the appends
    int rc = 0;
    for (Item &it : items) {
        const int n = it.io.num_tokens;
        if (n == 0) {
            it.len0 = nxt_kv_seq_len(st->index, it.seq);
            continue;
        }
        slots.assign((size_t)n, -1);
        if (it.seq < 0) {
            mapping.resize((size_t)n);
            src.resize((size_t)n);
            dst.resize((size_t)n);
            NxtKvAdmit a;
            const int r = nxt_kv_seq_admit(st->index, it.io.token_ids, n, mapping.data(),
                                           src.data(), dst.data(), &a);
            if (r != NXT_KV_OK) {
                rc = fail("exec: admitting %s failed (%d)", it.id.c_str(), r);
                break;
            }
            it.seq = a.seq;
            st->seqs[it.id] = a.seq;
            st->forget_device_row(a.seq);  // (a reused handle)
            // the prompt becomes shareable at once: later admissions (also in
            // this exec: their copies run after this exec's writes) find it
            nxt_kv_seq_cache(st->index, a.seq);
            slots = mapping;
            for (int c = 0; c < a.copy_count; ++c) {
                st->h_src.push(src[(size_t)c]);
                st->h_dst.push(dst[(size_t)c]);
            }
        } else {
            const int r = nxt_kv_seq_append(st->index, it.seq, it.io.token_ids, n, slots.data());
            if (r != NXT_KV_OK) {
                rc = fail("exec: appending to %s failed (%d)", it.id.c_str(), r);
                break;
            }
            it.len0 = nxt_kv_seq_len(st->index, it.seq) - n;
            it.open0 = opened.size();
            for (int t = 0; t < n; ++t) {
                const int pos = it.len0 + t;
                if (pos % s.block_size == 0)
                    opened.push_back({pos / s.block_size, slots[(size_t)t] / s.block_size});
            }
            it.nopen = opened.size() - it.open0;
        }
        for (int t = 0; t < n; ++t) {
            if (slots[(size_t)t] < 0) continue;
            st->h_slots.push(slots[(size_t)t]);
            st->h_kptr.push((const char *)it.io.key + (size_t)t * kv_row);
            st->h_vptr.push((const char *)it.io.value + (size_t)t * kv_row);
        }
    }

    tr.mark("index");
    // 2. the attention batch: requests with a query, their lengths, tables
    //    (the device-resident ones updated, or all of them uploaded) and groups
    st->h_seqs.n = st->h_qptr.n = st->h_optr.n = 0;
    st->h_bt.n = st->h_lens.n = st->h_group.n = st->h_pblocks.n = st->h_upd.n = 0;
    int width = 1, ng = 0, stride = 0;
    bool update = false;  // the device-resident tables are updated, not uploaded
    if (rc == 0 && (!st->h_lens.reserve(items.size()) || !st->h_len0.reserve(items.size())))
        rc = fail("exec: out of host memory");
    if (rc == 0) {
        st->h_len0.n = 0;
        for (const Item &it : items) {
            if (!it.io.query) continue;
            st->h_seqs.push(it.seq);
            st->h_qptr.push((const char *)it.io.query);
            st->h_optr.push((char *)it.io.output);
            const int len = nxt_kv_seq_len(st->index, it.seq);
            st->h_lens.p[st->h_lens.n++] = len;
            st->h_len0.p[st->h_len0.n++] = it.len0;
            width = std::max(width, (len + s.block_size - 1) / s.block_size);
        }
        const int B = (int)st->h_seqs.n;
        update = st->bt.can_update(st->h_seqs.p, st->h_len0.p, B, width);
        if (update) {
            stride = st->bt.stride;
            if (!st->h_upd.reserve(2 * opened.size() + 2)) {
                rc = fail("exec: out of host memory");
            } else {
                int i = 0;
                for (const Item &it : items) {
                    if (!it.io.query) continue;
                    for (size_t k = it.open0; k < it.open0 + it.nopen; ++k) {
                        st->h_upd.p[st->h_upd.n++] = st->bt.index(i, opened[k].first);
                        st->h_upd.p[st->h_upd.n++] = opened[k].second;
                    }
                    ++i;
                }
            }
        } else if (B > 0) {
            stride = xhip::ResidentTables::upload_stride(width, s.max_blocks);
            if (!st->h_bt.reserve((size_t)B * stride) ||
                !st->bt_dev.reserve((size_t)B * stride + 64)) {
                rc = fail("exec: out of memory");
            } else {
                st->h_bt.n = (size_t)B * stride;
                nxt_kv_batch_tables(st->index, st->h_seqs.p, B, stride, st->h_bt.p, st->h_lens.p);
            }
        }
        tr.mark(update ? "updates" : "tables");
        if (rc == 0 && B > 0) {
            if (!st->h_group.reserve((size_t)B) || !st->h_pblocks.reserve((size_t)B / 2 + 1)) {
                rc = fail("exec: out of host memory");
            } else if (update) {
                ng = st->bt.num_groups;
                st->h_group.n = st->bt.group.size();
                st->h_pblocks.n = st->bt.pblocks.size();
                std::memcpy(st->h_group.p, st->bt.group.data(), st->h_group.n * sizeof(int32_t));
                std::memcpy(st->h_pblocks.p, st->bt.pblocks.data(),
                            st->h_pblocks.n * sizeof(int32_t));
            } else {
                st->h_group.n = (size_t)B;
                nxt_kv_batch_prefix_groups(st->index, st->h_seqs.p, B, st->h_group.p,
                                           st->h_pblocks.p, &ng);
                st->h_pblocks.n = (size_t)std::max(ng, 1);
            }
        }
    }

    tr.mark("groups");
    // 3. one upload of everything the launches read, then the launches: the
    //    new rows, the copies of partly shared pages (a copy may read rows
    //    this exec writes), the query gather, the attention, the output scatter
    hipError_t e = hipSuccess;
    st->h_pack.n = 0;
    // (the tables first: the staging launch puts the pack's first
    // head_bytes into bt_dev and the rest into d_pack)
    st->pack(st->h_bt);
    const size_t head_bytes = st->h_bt.n ? (st->h_pack.n + 255) & ~(size_t)255 : 0;
    const size_t o_slots = st->pack(st->h_slots), o_kptr = st->pack(st->h_kptr),
                 o_vptr = st->pack(st->h_vptr), o_src = st->pack(st->h_src),
                 o_dst = st->pack(st->h_dst), o_lens = st->pack(st->h_lens),
                 o_group = st->pack(st->h_group), o_pblocks = st->pack(st->h_pblocks),
                 o_qptr = st->pack(st->h_qptr), o_optr = st->pack(st->h_optr);
    tr.mark("pack");
    // The rows of requests admitted or extended before a failure are still
    // written: the index already holds their tokens.
    bool staged = false;
    char *const hp = st->h_pack.p;
    xhip::KvAppendParams p;
    std::memset(&p, 0, sizeof(p));
    p.key_cache = st->key_cache;
    p.value_cache = st->value_cache;
    p.kv_block_stride_bytes = (long long)s.num_kv_heads * s.block_size * s.head_size * s.elem_bytes;
    p.kv_head_stride_bytes = (long long)s.block_size * s.head_size * s.elem_bytes;
    p.num_kv_heads = s.num_kv_heads;
    p.row_bytes = s.head_size * s.elem_bytes;
    p.row_chunks = p.row_bytes / 16;
    p.block_size = s.block_size;
    p.bs_shift = __builtin_ctz((unsigned)s.block_size);
    // The staging copy, and in the same launch the new tokens' K/V rows,
    // whose slots and row pointers that launch reads from the host-pinned
    // pack (launch_stage_copy_append).
    xhip::StageTables tables;
    tables.head = st->bt_dev.p;
    tables.head_bytes = (long long)head_bytes;
    tables.pairs = st->h_upd.p;
    tables.count = (int)(st->h_upd.n / 2);
    tables.table = st->bt_dev.p;
    if (st->h_pack.n == (size_t)-1) {
        rc = fail("exec: out of host memory");
    } else if (head_bytes && st->h_pack.n <= head_bytes) {
        rc = fail("exec: staging layout");  // (the lengths always follow the tables)
    } else if (st->h_pack.n > 0) {
        const size_t bytes = (st->h_pack.n + 15) & ~(size_t)15;
        if (!st->d_pack.reserve(bytes - head_bytes)) {
            rc = fail("exec: out of device memory");
        } else {
            if (st->h_slots.n) {
                xhip::KvAppendParams w = p;
                w.slots = (const int *)(hp + o_slots);
                w.key_rows = (const char *const *)(hp + o_kptr);
                w.value_rows = (const char *const *)(hp + o_vptr);
                w.num_tokens = (int)st->h_slots.n;
                e = xhip::launch_stage_copy_append(st->d_pack.p, hp, bytes, w, st->stream,
                                                   &tables);
            } else {
                e = xhip::launch_stage_copy(st->d_pack.p, hp, bytes, st->stream, &tables);
            }
            staged = e == hipSuccess;
        }
    }
    // device address of the part at pack offset `off` (every part but the
    // tables lies past head_bytes)
    char *const dp = st->d_pack.p;
    auto at = [dp, head_bytes](size_t off) { return (void *)(dp + (off - head_bytes)); };
    if (staged && e == hipSuccess && st->h_src.n) {
        xhip::KvAppendParams c = p;
        c.key = st->key_cache;
        c.value = st->value_cache;
        c.slots = (const int *)at(o_dst);
        c.src_slots = (const int *)at(o_src);
        c.num_tokens = (int)st->h_src.n;
        e = xhip::launch_kv_append(c, st->stream);
    }
    if (e != hipSuccess) rc = fail("exec: K/V write: %s", hipGetErrorString(e));
    const int B = (int)st->h_seqs.n;
    if (rc == 0 && staged && B > 0) {
        // the attention reads each request's query rows and writes its output
        // rows in place, through the staged row pointer tables
        const int kbs = s.num_kv_heads * s.block_size * s.head_size;
        const int khs = s.block_size * s.head_size;
        const int *bt = st->bt_dev.p, *lens = (const int *)at(o_lens);
        const char *const *qr = (const char *const *)at(o_qptr);
        char *const *orw = (char *const *)at(o_optr);
        const int a =
            ng > 0 ? xhip_paged_attention_cascade_rows(
                         qr, orw, st->key_cache, st->value_cache, bt, lens,
                         (const int *)at(o_group), (const int *)at(o_pblocks), ng, B, s.num_heads,
                         s.head_size, s.num_kv_heads, s.scale, stride, s.block_size, kbs, khs,
                         s.kv_dtype, st->stream)
                   : xhip_paged_attention_rows(qr, orw, st->key_cache, st->value_cache, bt, lens,
                                               B, s.num_heads, s.head_size, s.num_kv_heads,
                                               s.scale, stride, s.block_size, kbs, khs,
                                               s.kv_dtype, st->stream);
        if (a != NXT_ATTN_OK) rc = fail("exec: attention: %s", nxt_attn_last_error());
    }
    // what the device-resident tables now hold
    if (B > 0 || rc != 0)
        st->bt.commit(rc == 0 && staged, !update, st->h_seqs.p, st->h_lens.p, B, stride,
                      st->h_group.p, st->h_group.n, st->h_pblocks.p, st->h_pblocks.n, ng);
    return rc;
}

// One exec of the requests `ids` (in order): the whole-batch decode step.
int exec_ids(NxtModelInstance *instance, InstanceState *st, const std::vector<std::string> &ids) {
    const ModelSpec &s = st->spec;
    const uint32_t request_count = (uint32_t)ids.size();
    const auto t0 = std::chrono::steady_clock::now();
    PhaseTrace tr(t0);
    if ((int)request_count > s.max_batch)
        return fail("exec: %u requests > max_batch_size %d", request_count, s.max_batch);

    // every request bound, each once (a bound entry carries the stamp of the
    // exec that took it)
    std::vector<Item> items;
    items.reserve(request_count);
    const uint64_t stamp = ++st->exec_stamp;
    for (uint32_t i = 0; i < request_count; ++i) {
        const std::string &id = ids[i];
        auto b = st->bound.find(id);
        if (b == st->bound.end()) return fail("exec: request %s has no bound buffers", id.c_str());
        if (b->second.exec_stamp == stamp)
            return fail("exec: request %s twice in one batch", id.c_str());
        b->second.exec_stamp = stamp;
        auto q = st->seqs.find(id);
        items.push_back({id, b->second.io, q == st->seqs.end() ? -1 : q->second});
        if (items.back().seq < 0 && b->second.io.num_tokens == 0)
            return fail("exec: new request %s without tokens", id.c_str());
    }
    if (hipSetDevice(st->device) != hipSuccess) return fail("exec: hipSetDevice failed");

    tr.mark("validate");
    int rc = fast_ok(st, items) ? fast_step(st, items[0]) : slow_step(st, items, tr);
    tr.mark("launch");
    // the bindings are consumed (the items hold what the exec needs), while
    // the device works
    for (const Item &it : items) st->bound.erase(it.id);
    // wait for the device (wait_exec: the completion word; polling
    // hipStreamQuery instead of hipStreamSynchronize took 6-8 us longer per
    // exec), then end the released requests
    const hipError_t e = wait_exec(st);
    if (e != hipSuccess && rc == 0) rc = fail("exec: %s", hipGetErrorString(e));
    if (rc != 0)  // what the device holds of the exec's sequences is unknown
        for (const Item &it : items) st->forget_device_row(it.seq);
    for (const Item &it : items) {
        if (rc == 0 && it.io.release && it.seq >= 0) {
            nxt_kv_seq_release(st->index, it.seq, 1);
            st->forget_device_row(it.seq);  // its handle may be reused
            st->seqs.erase(it.id);
        }
    }
    instance->exec_count++;
    tr.mark("wait");
    tr.report(request_count);
    instance->total_exec_ms +=
        std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    return rc;
}

}  // namespace
