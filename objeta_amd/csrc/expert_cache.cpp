// expert_cache.cpp — single-GPU VRAM expert cache and the host-in/host-out
// selected-expert MoE executor.
//
// Cache semantics follow CudaExpertCache (crates/objeta-cuda/src/moe.rs:70-226):
// an LRU order over tensors, pinned entries that eviction skips, an insert that
// bypasses tensors larger than the capacity, and the reference's counters.
// Differences of mechanism, not of semantics:
//   * LRU lookups are O(1) (list + iterator map) instead of Vec scans.
//   * Device memory is recycled, not freed: an evicted tensor's block returns to a
//     size-keyed free list together with events recorded on every stream of the
//     context at the moment it was released; a later insert of the same size makes
//     its copy stream wait for those events, so the block is never overwritten
//     while a kernel enqueued before the eviction may still read it. The reference
//     gets the same guarantee from Arc + stream-ordered frees (moe.rs:117,155).
//   * Blocks referenced by an executor call in flight are not recycled until the
//     call releases them (the reference's Arc clones held by the executor).
//   * When only pinned entries remain, insert stops evicting and admits the tensor
//     over capacity instead of looping forever (moe.rs:145-147).
//
// The executor follows execute_selected_moe_cuda (moe.rs:352-751) and
// execute_selected_moe_native_fp4_cuda (moe.rs:816-1280): same validation,
// admission, cache keys and byte accounting, but the weight copies of misses go
// to the context's copy stream from the caller's host memory, and each expert's
// fused kernels wait only for its own copies, so copies overlap compute. With no
// misses the call is one fused launch pair for all selected experts.
#include <algorithm>
#include <chrono>
#include <cstring>
#include <deque>
#include <list>
#include <map>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "host_common.hpp"
#include "kernels.hpp"

namespace objeta {
namespace {

struct Key {
    uint64_t layer, expert;
    int32_t kind, fmt;
    bool operator==(const Key& o) const {
        return layer == o.layer && expert == o.expert && kind == o.kind && fmt == o.fmt;
    }
};
struct KeyHash {
    size_t operator()(const Key& k) const {
        uint64_t h = k.layer * 0x9E3779B97F4A7C15ull ^ (k.expert + 0x632BE59BD9B4E019ull);
        h ^= (static_cast<uint64_t>(static_cast<uint32_t>(k.kind)) << 32) | static_cast<uint32_t>(k.fmt);
        h ^= h >> 29;
        return static_cast<size_t>(h * 0xBF58476D1CE4E5B9ull);
    }
};
Key to_key(const objeta_hip_cache_key& k) { return Key{k.layer_id, k.expert_id, k.tensor_kind, k.quant_format}; }
objeta_hip_cache_key from_key(const Key& k) {
    objeta_hip_cache_key o{};
    o.layer_id = k.layer;
    o.expert_id = k.expert;
    o.tensor_kind = k.kind;
    o.quant_format = k.fmt;
    return o;
}

struct Block {
    void* ptr = nullptr;
    size_t bytes = 0;
    int refs = 0;          // executor references of a call in flight
    bool in_cache = false;  // owned by a cache entry
    bool carved = false;    // inside one of the cache's chunks (freed with the chunk)
    std::vector<hipEvent_t> fence;
    hipEvent_t ready = nullptr;  // recorded on the copy stream after the fill; NULL once known complete
    // The reads since the fill: per stream, the mark that ends the last library call
    // that used the block there (0: no mark, fence at reuse); and, once its pointer went
    // out through the cache API (the caller's streams are not known), every stream of
    // the context.
    std::vector<std::pair<hipStream_t, uint64_t>> last_use;
    bool all_streams = true;
};

}  // namespace
}  // namespace objeta

struct objeta_hip_expert_cache {
    objeta_hip_context* ctx = nullptr;  // NULL: accounting only
    objeta_hip_cache_stats st{};
    struct Entry {
        objeta::Block* blk;
        size_t size;
        std::list<objeta::Key>::iterator pos;
    };
    std::unordered_map<objeta::Key, Entry, objeta::KeyHash> map;
    std::list<objeta::Key> order;  // front = least recently used
    std::unordered_set<objeta::Key, objeta::KeyHash> pinned;
    std::multimap<size_t, objeta::Block*> free_blocks;  // recycled, fenced
    std::unordered_map<const void*, objeta::Block*> transients;
    std::vector<hipEvent_t> event_pool;
    size_t free_bytes = 0;
    size_t device_bytes = 0;  // all device memory allocated by this cache
    struct Chunk {
        char* base;
        size_t size, used;
    };
    std::vector<Chunk> chunks;  // blocks are carved from these (see acquire_block)
    // Per stream, the events that end the library's calls on it (the context's transient
    // pool keeps these): mark n is done once its event has completed.
    struct UseLog {
        uint64_t next = 1, done = 0;
        std::deque<std::pair<uint64_t, hipEvent_t>> pending;
    };
    std::unordered_map<hipStream_t, UseLog> uses;
};

namespace objeta {
namespace {

using Cache = objeta_hip_expert_cache;

size_t free_list_cap(const Cache* c) {
    const size_t floor = size_t(64) << 20;
    return c->st.capacity_bytes > floor ? static_cast<size_t>(c->st.capacity_bytes) : floor;
}

hipEvent_t take_event(Cache* c) {
    if (!c->event_pool.empty()) {
        hipEvent_t e = c->event_pool.back();
        c->event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return e;
}

Cache* transient_pool(objeta_hip_context* ctx);

// Retires the completed marks of `u` up to `id`, oldest first (the marks of one stream
// complete in order); their events go back to `log`'s pool.
void retire_marks(Cache* log, Cache::UseLog& u, uint64_t id) {
    while (u.done < id && !u.pending.empty()) {
        const hipError_t q = hipEventQuery(u.pending.front().second);
        if (q != hipSuccess) {
            if (q != hipErrorNotReady) (void)hipGetLastError();
            break;
        }
        u.done = u.pending.front().first;
        log->event_pool.push_back(u.pending.front().second);
        u.pending.pop_front();
    }
}

// A new mark on `s` in `log`'s use log: an event recorded after the work enqueued so
// far (the completed older marks are retired first, so the log stays short). 0 when
// the record failed.
uint64_t mark_use(Cache* log, hipStream_t s) {
    auto& u = log->uses[s];
    retire_marks(log, u, u.next);
    hipEvent_t e = take_event(log);
    if (!e) return 0;
    if (hipEventRecord(e, s) != hipSuccess) {
        (void)hipGetLastError();
        log->event_pool.push_back(e);
        return 0;
    }
    u.pending.emplace_back(u.next, e);
    return u.next++;
}

// Whether the work before mark `id` on `s` has completed.
bool use_done(Cache* log, hipStream_t s, uint64_t id) {
    auto it = log->uses.find(s);
    if (id == 0 || it == log->uses.end()) return false;
    retire_marks(log, it->second, id);
    return it->second.done >= id;
}

// Records, on every stream whose reads of `b` may still be running, the point after
// which `b` is free: a read by a library call whose mark has completed needs no fence.
// The copy stream needs none: every fill of a block is a copy on it, so a refill
// follows the last fill in stream order, and `ready` (kept) still marks that fill's
// end for destroy_block.
void fence_block(Cache* c, Block* b) {
    for (hipEvent_t e : b->fence) c->event_pool.push_back(e);
    b->fence.clear();
    if (!c->ctx) return;
    auto rec = [&](hipStream_t s) {
        hipEvent_t e = take_event(c);
        if (e && hipEventRecord(e, s) == hipSuccess) {
            b->fence.push_back(e);
            return;
        }
        (void)hipGetLastError();
        if (e) c->event_pool.push_back(e);
    };
    if (b->all_streams)
        for (hipStream_t s : c->ctx->streams) rec(s);
    Cache* log = transient_pool(c->ctx);
    for (const auto& u : b->last_use) {
        if (b->all_streams &&
            std::find(c->ctx->streams.begin(), c->ctx->streams.end(), u.first) != c->ctx->streams.end())
            continue;  // fenced above
        if (!use_done(log, u.first, u.second)) rec(u.first);
    }
    b->last_use.clear();
}

// The block's pointer went out through the cache API: its readers are not known.
void use_block_anywhere(Block* b) { b->all_streams = true; }

// A library call on `s` that read `b` ends at mark `id` (kept also for a block handed
// out through the API: `s` may be a stream outside the context).
void set_last_use(Block* b, hipStream_t s, uint64_t id) {
    for (auto& u : b->last_use)
        if (u.first == s) {
            u.second = id;
            return;
        }
    b->last_use.emplace_back(s, id);
}

void destroy_block(Cache* c, Block* b) {
    if (c->ctx && b->ptr) {
        for (hipEvent_t e : b->fence) (void)hipEventSynchronize(e);
        if (b->ready) (void)hipEventSynchronize(b->ready);
        if (!b->carved) {  // a carved block's bytes stay with its chunk
            (void)hipFree(b->ptr);
            c->device_bytes -= b->bytes;
        }
    }
    for (hipEvent_t e : b->fence) c->event_pool.push_back(e);
    if (b->ready) c->event_pool.push_back(b->ready);
    delete b;
}

// A block left the cache or a call: recycle it once nothing references it.
void retire_block(Cache* c, Block* b) {
    if (b->in_cache || b->refs > 0) return;
    fence_block(c, b);
    c->free_blocks.emplace(b->bytes, b);
    c->free_bytes += b->bytes;
    while (c->free_bytes > free_list_cap(c) && !c->free_blocks.empty()) {
        auto it = c->free_blocks.begin();  // smallest first
        Block* v = it->second;
        c->free_blocks.erase(it);
        c->free_bytes -= v->bytes;
        destroy_block(c, v);
    }
}

// Blocks come from 64 MiB chunks, carved in order: a miss then costs no hipMalloc
// (about 50-100 us each on MI355X, several per layer while a cache fills). A carved
// block is recycled through the free lists like any other, but its bytes return to
// the device only with its chunk, when the cache releases its memory; carving stops
// once the chunks hold the capacity plus the free lists' cap, and blocks past that
// are allocated one by one as before.
constexpr size_t kChunkBytes = size_t(64) << 20;

bool carve_block(Cache* c, Block* b) {
    const size_t need = (b->bytes + 255) & ~size_t(255);
    if (c->chunks.empty() || c->chunks.back().size - c->chunks.back().used < need) {
        size_t held = 0;
        for (const auto& ch : c->chunks) held += ch.size;
        const size_t size = need > kChunkBytes ? need : kChunkBytes;
        if (held + size > static_cast<size_t>(c->st.capacity_bytes) + free_list_cap(c)) return false;
        void* p = nullptr;
        if (hipMalloc(&p, size) != hipSuccess) {
            (void)hipGetLastError();
            return false;
        }
        c->chunks.push_back({static_cast<char*>(p), size, 0});
        c->device_bytes += size;
    }
    auto& ch = c->chunks.back();
    b->ptr = ch.base + ch.used;
    b->carved = true;
    ch.used += need;
    return true;
}

// A block of exactly `bytes` whose previous contents may be overwritten by work
// enqueued on `s` from now on.
int32_t acquire_block(Cache* c, size_t bytes, hipStream_t s, Block** out) {
    auto it = c->free_blocks.find(bytes);
    if (it != c->free_blocks.end()) {
        Block* b = it->second;
        c->free_blocks.erase(it);
        c->free_bytes -= b->bytes;
        for (hipEvent_t e : b->fence) {  // a fence already passed needs no wait
            const hipError_t q = hipEventQuery(e);
            if (q == hipSuccess) continue;
            if (q != hipErrorNotReady) (void)hipGetLastError();
            OBJ_HIP(hipStreamWaitEvent(s, e, 0), "fence recycled cache block");
        }
        *out = b;
        return 0;
    }
    Block* b = new Block();
    b->bytes = bytes;
    if (c->ctx && bytes && carve_block(c, b)) {
        *out = b;
        return 0;
    }
    if (c->ctx && bytes) {
        hipError_t e = hipMalloc(&b->ptr, bytes);
        if (e != hipSuccess && !c->free_blocks.empty()) {
            (void)hipGetLastError();
            while (!c->free_blocks.empty()) {  // give recycled memory back and retry
                auto v = c->free_blocks.begin();
                Block* blk = v->second;
                c->free_blocks.erase(v);
                c->free_bytes -= blk->bytes;
                destroy_block(c, blk);
            }
            e = hipMalloc(&b->ptr, bytes);
        }
        if (e != hipSuccess) {
            (void)hipGetLastError();
            delete b;
            OBJ_FAIL(kDriver, strf("allocate cache block of %zu bytes", bytes), hipGetErrorString(e));
        }
        c->device_bytes += bytes;
    }
    *out = b;
    return 0;
}

// The pinned-source copies of one call, launched together by flush_copies; each
// block's ready event is recorded after that launch. `key` names the cache entry a
// block was inserted under (keyed), so that a failed launch can take it out again.
struct CopyBatch {
    struct Pending {
        Cache* c;
        Block* b;
        Key key;
        bool keyed;
    };
    std::vector<H2dCopy> copies;
    std::vector<Pending> blocks;
    ~CopyBatch();  // takes out the entries of copies never launched (an error on the way)
};

// Copies host bytes into a block on the copy stream, ordered after `s` (s NULL: after
// nothing but earlier copy-stream work, for prefetches), and records the block's
// ready event after the copy. With `batch`, a pinned source's copy is added to it
// instead (launched, and the ready event recorded, by flush_copies).
int32_t fill_block(Cache* c, Block* b, const void* h_src, size_t n, hipStream_t s, CopyBatch* batch = nullptr) {
    if (!c->ctx || n == 0) return 0;
    if (!h_src) OBJ_FAIL(kInvalidInput, "copy tensor into the cache", "NULL host pointer");
    b->last_use.clear();  // new contents: no reader yet
    b->all_streams = false;
    hipStream_t cs = c->ctx->copy_stream;
    hipError_t r = hipSuccess;
    if (s) {
        hipEvent_t e = take_event(c);
        if (!e) OBJ_FAIL(kDriver, "copy tensor into the cache", "event creation failed");
        r = hipEventRecord(e, s);
        if (r == hipSuccess) r = hipStreamWaitEvent(cs, e, 0);
        c->event_pool.push_back(e);
    }
    // pinned sources by a kernel (a DMA copy behind a cross-stream wait starts late)
    const void* dsrc = r == hipSuccess ? pinned_device_ptr(h_src, n) : nullptr;
    if (dsrc && batch) {
        batch->copies.push_back(H2dCopy{b->ptr, dsrc, n});
        batch->blocks.push_back(CopyBatch::Pending{c, b, Key{}, false});
        return 0;
    }
    if (dsrc) OBJ_TRY(launch_h2d_copy(cs, b->ptr, dsrc, n));
    else if (r == hipSuccess) r = hipMemcpyAsync(b->ptr, h_src, n, hipMemcpyHostToDevice, cs);
    if (r == hipSuccess) {
        if (b->ready) c->event_pool.push_back(b->ready);
        b->ready = take_event(c);
        if (!b->ready) OBJ_FAIL(kDriver, "copy tensor into the cache", "event creation failed");
        r = hipEventRecord(b->ready, cs);
    }
    if (r != hipSuccess) {
        (void)hipGetLastError();
        OBJ_FAIL(kDriver, "copy tensor into the cache", hipGetErrorString(r));
    }
    return 0;
}

// Orders work enqueued on `s` from now on after the block's fill (a prefetch or an
// insert made for another stream may still be copying). s NULL: waits on the host.
int32_t wait_ready(Cache* c, Block* b, hipStream_t s) {
    if (!b->ready) return 0;
    hipError_t r = hipEventQuery(b->ready);
    if (r == hipSuccess) {
        c->event_pool.push_back(b->ready);
        b->ready = nullptr;
        return 0;
    }
    if (r != hipErrorNotReady) {
        (void)hipGetLastError();
        OBJ_FAIL(kDriver, "wait for a cache copy", hipGetErrorString(r));
    }
    OBJ_HIP(s ? hipStreamWaitEvent(s, b->ready, 0) : hipEventSynchronize(b->ready), "wait for a cache copy");
    if (!s) {
        c->event_pool.push_back(b->ready);
        b->ready = nullptr;
    }
    return 0;
}

// Makes `s` wait for everything enqueued so far on the copy stream.
int32_t join_copies(Cache* c, hipStream_t s) {
    if (!c || !c->ctx) return 0;
    hipEvent_t e = take_event(c);
    if (!e) OBJ_FAIL(kDriver, "join cache copies", "event creation failed");
    hipError_t r = hipEventRecord(e, c->ctx->copy_stream);
    if (r == hipSuccess) r = hipStreamWaitEvent(s, e, 0);
    c->event_pool.push_back(e);
    if (r != hipSuccess) {
        (void)hipGetLastError();
        OBJ_FAIL(kDriver, "join cache copies", hipGetErrorString(r));
    }
    return 0;
}

void touch(Cache* c, const Key& k) {  // moe.rs:160-165
    auto it = c->map.find(k);
    if (it == c->map.end()) return;
    c->order.splice(c->order.end(), c->order, it->second.pos);
}

bool evict_lru(Cache* c, Key* out) {  // moe.rs:167-180
    for (auto it = c->order.begin(); it != c->order.end(); ++it) {
        if (c->pinned.count(*it)) continue;
        const Key k = *it;
        c->order.erase(it);
        auto m = c->map.find(k);
        Block* b = m->second.blk;
        c->st.resident_bytes -= m->second.size;
        c->st.eviction_count += 1;
        c->map.erase(m);
        b->in_cache = false;
        retire_block(c, b);
        if (out) *out = k;
        return true;
    }
    return false;
}

void remove_existing(Cache* c, const Key& k) {
    auto m = c->map.find(k);
    if (m == c->map.end()) return;
    c->st.resident_bytes -= m->second.size;
    c->order.erase(m->second.pos);
    Block* b = m->second.blk;
    c->map.erase(m);
    b->in_cache = false;
    retire_block(c, b);
}

CopyBatch::~CopyBatch() {
    for (const auto& p : blocks) {
        if (!p.keyed) continue;
        auto m = p.c->map.find(p.key);
        if (m != p.c->map.end() && m->second.blk == p.b) remove_existing(p.c, p.key);
    }
}

void make_room(Cache* c, size_t size) {
    while (c->st.resident_bytes + size > c->st.capacity_bytes && !c->order.empty())
        if (!evict_lru(c, nullptr)) break;
}

Block* lookup(Cache* c, const Key& k) {  // get (moe.rs:113-122)
    auto it = c->map.find(k);
    if (it == c->map.end()) {
        c->st.miss_count += 1;
        return nullptr;
    }
    c->st.hit_count += 1;
    c->order.splice(c->order.end(), c->order, it->second.pos);
    return it->second.blk;
}

// insert (moe.rs:124-158) of a filled block. Returns false (block untouched and
// still owned by the caller) when the tensor is larger than the capacity.
bool insert_block(Cache* c, const Key& k, Block* b, size_t size) {
    c->st.cache_insert_attempt_count += 1;
    if (size > c->st.capacity_bytes) {
        c->st.oversized_tensor_bypass_count += 1;
        c->st.cache_insert_bypass_count += 1;
        return false;
    }
    c->st.cache_insert_accept_count += 1;
    remove_existing(c, k);
    make_room(c, size);
    c->order.push_back(k);
    b->in_cache = true;
    c->map.emplace(k, Cache::Entry{b, size, std::prev(c->order.end())});
    c->st.resident_bytes += size;
    return true;
}

// A filled block for host bytes: recycled or new, copy enqueued after `s` (or added to
// `batch`).
int32_t stage_tensor(Cache* c, const void* h_src, size_t n, hipStream_t s, Block** out, CopyBatch* batch = nullptr) {
    Block* b = nullptr;
    OBJ_TRY(acquire_block(c, n, c->ctx ? c->ctx->copy_stream : nullptr, &b));
    int32_t rc = fill_block(c, b, h_src, n, s, batch);
    if (rc) {
        retire_block(c, b);
        return rc;
    }
    *out = b;
    return 0;
}

// Launches the batch's copies on the copy stream and records each block's ready event
// after them. On failure the error is returned with the batch left full, and its
// destructor takes the blocks' cache entries out (their bytes may not have arrived).
int32_t flush_copies(objeta_hip_context* ctx, CopyBatch& batch) {
    if (batch.copies.empty()) return 0;
    int32_t rc = launch_h2d_copy_batch(ctx->copy_stream, batch.copies.data(), batch.copies.size());
    for (size_t i = 0; i < batch.blocks.size() && rc == 0; ++i) {
        Cache* c = batch.blocks[i].c;
        Block* b = batch.blocks[i].b;
        if (b->ready) c->event_pool.push_back(b->ready);
        b->ready = take_event(c);
        if (!b->ready || hipEventRecord(b->ready, ctx->copy_stream) != hipSuccess) {
            (void)hipGetLastError();
            rc = set_error(kDriver, __FILE__, __LINE__, __func__, "copy tensor into the cache", "event failure");
        }
    }
    if (rc) {
        (void)hipStreamSynchronize(ctx->copy_stream);
        return rc;  // the batch's destructor takes the entries out
    }
    batch.copies.clear();
    batch.blocks.clear();
    return 0;
}

int32_t check_cache(const objeta_hip_expert_cache* c, const char* action) {
    if (!c) OBJ_FAIL(kInvalidInput, action, "cache is NULL");
    return 0;
}

// Frees every device block and event of `c` (the context is going away).
void release_device(Cache* c) {
    if (!c->ctx) return;
    std::vector<Block*> all;
    for (auto& kv : c->map) all.push_back(kv.second.blk);
    for (auto& kv : c->free_blocks) all.push_back(kv.second);
    for (auto& kv : c->transients) all.push_back(kv.second);
    for (Block* b : all) destroy_block(c, b);
    // a carved block still held by a call in flight is in none of the lists above: wait
    // for the device before its chunk goes
    if (!c->chunks.empty()) (void)hipDeviceSynchronize();
    for (const auto& ch : c->chunks) (void)hipFree(ch.base);
    c->device_bytes = 0;
    c->chunks.clear();
    c->map.clear();
    c->order.clear();
    c->pinned.clear();
    c->free_blocks.clear();
    c->transients.clear();
    c->free_bytes = 0;
    c->st.resident_bytes = 0;
    c->st.pinned_bytes = 0;
    for (auto& kv : c->uses)
        for (auto& pe : kv.second.pending) c->event_pool.push_back(pe.second);
    c->uses.clear();
    for (hipEvent_t e : c->event_pool) (void)hipEventDestroy(e);
    c->event_pool.clear();
    c->ctx = nullptr;
}

}  // namespace

void detach_caches(objeta_hip_context* ctx) {
    for (void* p : ctx->caches) release_device(static_cast<Cache*>(p));
    ctx->caches.clear();
}

}  // namespace objeta

using namespace objeta;

extern "C" {

int32_t objeta_hip_cache_create(objeta_hip_context* ctx, uint64_t capacity_bytes, objeta_hip_expert_cache** out) {
    OBJ_GUARD_BEGIN
    if (!out) OBJ_FAIL(kInvalidInput, "create expert cache", "out is NULL");
    auto* c = new objeta_hip_expert_cache();
    c->ctx = ctx;
    c->st.capacity_bytes = capacity_bytes;
    if (ctx) ctx->caches.push_back(c);
    *out = c;
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_cache_destroy(objeta_hip_expert_cache* c) {
    OBJ_GUARD_BEGIN
    if (!c) return 0;
    if (c->ctx) {
        objeta_hip_context* ctx = c->ctx;
        (void)hipSetDevice(ctx->device);
        for (hipStream_t s : ctx->streams) (void)hipStreamSynchronize(s);
        (void)hipStreamSynchronize(ctx->copy_stream);
        auto& v = ctx->caches;
        v.erase(std::remove(v.begin(), v.end(), static_cast<void*>(c)), v.end());
        release_device(c);
    } else {
        std::vector<Block*> all;
        for (auto& kv : c->map) all.push_back(kv.second.blk);
        for (auto& kv : c->free_blocks) all.push_back(kv.second);
        for (auto& kv : c->transients) all.push_back(kv.second);
        for (Block* b : all) destroy_block(c, b);
    }
    delete c;
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_cache_stats_get(const objeta_hip_expert_cache* c, objeta_hip_cache_stats* out) {
    OBJ_TRY(check_cache(c, "cache stats"));
    if (!out) OBJ_FAIL(kInvalidInput, "cache stats", "out is NULL");
    *out = c->st;
    out->entry_count = c->map.size();
    out->device_bytes_reserved = c->device_bytes;
    return 0;
}

int32_t objeta_hip_cache_set_bypass_oversized_experts(objeta_hip_expert_cache* c, int32_t enable) {
    OBJ_TRY(check_cache(c, "set bypass_oversized_experts"));
    c->st.bypass_oversized_experts = enable ? 1 : 0;
    return 0;
}

int32_t objeta_hip_cache_get(objeta_hip_expert_cache* c, const objeta_hip_cache_key* key, int32_t* hit,
                             const void** d_ptr, uint64_t* nbytes) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_cache(c, "cache get"));
    if (!key || !hit) OBJ_FAIL(kInvalidInput, "cache get", "NULL argument");
    Block* b = lookup(c, to_key(*key));
    *hit = b ? 1 : 0;
    if (b && c->ctx) OBJ_TRY(wait_ready(c, b, nullptr));  // a prefetch may still be copying
    if (b) use_block_anywhere(b);  // the pointer leaves the library
    if (d_ptr) *d_ptr = b ? b->ptr : nullptr;
    if (nbytes) *nbytes = b ? c->map.find(to_key(*key))->second.size : 0;
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_cache_insert(objeta_hip_expert_cache* c, const objeta_hip_cache_key* key, const void* h_src,
                                uint64_t nbytes, objeta_hip_stream stream, const void** d_ptr, int32_t* cached) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_cache(c, "cache insert"));
    if (!key || !d_ptr || !cached) OBJ_FAIL(kInvalidInput, "cache insert", "NULL argument");
    hipStream_t s = nullptr;
    if (c->ctx) {
        OBJ_HIP(hipSetDevice(c->ctx->device), "hipSetDevice");
        s = resolve_stream(c->ctx, stream);
    }
    Block* b = nullptr;
    OBJ_TRY(stage_tensor(c, h_src, nbytes, s, &b));
    if (c->ctx) OBJ_TRY(join_copies(c, s));
    const bool ok = insert_block(c, to_key(*key), b, nbytes);
    use_block_anywhere(b);  // the pointer leaves the library
    if (!ok && b->ptr) c->transients[b->ptr] = b;
    else if (!ok) retire_block(c, b);
    *cached = ok ? 1 : 0;
    *d_ptr = b->ptr;
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_cache_get_or_insert(objeta_hip_expert_cache* c, const objeta_hip_cache_key* key,
                                       const void* h_src, uint64_t nbytes, objeta_hip_stream stream,
                                       const void** d_ptr, int32_t* hit, int32_t* cached) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_cache(c, "cache get_or_insert"));
    if (!key || !d_ptr || !hit || !cached) OBJ_FAIL(kInvalidInput, "cache get_or_insert", "NULL argument");
    Block* b = lookup(c, to_key(*key));
    if (b) {
        if (c->ctx) {
            hipStream_t s = resolve_stream(c->ctx, stream);
            OBJ_TRY(wait_ready(c, b, s));
        }
        use_block_anywhere(b);  // the pointer leaves the library
        *hit = 1;
        *cached = 1;
        *d_ptr = b->ptr;
        return 0;
    }
    *hit = 0;
    return objeta_hip_cache_insert(c, key, h_src, nbytes, stream, d_ptr, cached);
    OBJ_GUARD_END
}

int32_t objeta_hip_cache_insert_pinned(objeta_hip_expert_cache* c, const objeta_hip_cache_key* key,
                                       const void* h_src, uint64_t nbytes, objeta_hip_stream stream,
                                       const void** d_ptr) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_cache(c, "cache insert_pinned"));
    if (!key || !d_ptr) OBJ_FAIL(kInvalidInput, "cache insert_pinned", "NULL argument");
    hipStream_t s = nullptr;
    if (c->ctx) {
        OBJ_HIP(hipSetDevice(c->ctx->device), "hipSetDevice");
        s = resolve_stream(c->ctx, stream);
    }
    const Key k = to_key(*key);
    make_room(c, nbytes);  // moe.rs:195-199
    Block* b = nullptr;
    OBJ_TRY(stage_tensor(c, h_src, nbytes, s, &b));
    if (c->ctx) OBJ_TRY(join_copies(c, s));
    remove_existing(c, k);
    c->order.push_back(k);
    b->in_cache = true;
    c->map.emplace(k, Cache::Entry{b, nbytes, std::prev(c->order.end())});
    c->st.resident_bytes += nbytes;
    c->st.pinned_bytes += nbytes;
    c->pinned.insert(k);
    use_block_anywhere(b);  // the pointer leaves the library
    *d_ptr = b->ptr;
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_cache_pin(objeta_hip_expert_cache* c, const objeta_hip_cache_key* key) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_cache(c, "cache pin"));
    if (!key) OBJ_FAIL(kInvalidInput, "cache pin", "key is NULL");
    const Key k = to_key(*key);
    auto it = c->map.find(k);
    if (it != c->map.end() && !c->pinned.count(k)) {
        c->pinned.insert(k);
        c->st.pinned_bytes += it->second.size;
    }
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_cache_touch(objeta_hip_expert_cache* c, const objeta_hip_cache_key* key) {
    OBJ_TRY(check_cache(c, "cache touch"));
    if (!key) OBJ_FAIL(kInvalidInput, "cache touch", "key is NULL");
    touch(c, to_key(*key));
    return 0;
}

int32_t objeta_hip_cache_evict_lru(objeta_hip_expert_cache* c, int32_t* evicted, objeta_hip_cache_key* key_out) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_cache(c, "cache evict_lru"));
    if (!evicted) OBJ_FAIL(kInvalidInput, "cache evict_lru", "NULL argument");
    Key k{};
    *evicted = evict_lru(c, &k) ? 1 : 0;
    if (*evicted && key_out) *key_out = from_key(k);
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_cache_clear(objeta_hip_expert_cache* c) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_cache(c, "cache clear"));
    std::vector<Block*> blocks;
    for (auto& kv : c->map) blocks.push_back(kv.second.blk);
    c->map.clear();
    c->order.clear();
    c->pinned.clear();
    c->st.resident_bytes = 0;
    c->st.pinned_bytes = 0;
    for (Block* b : blocks) {
        b->in_cache = false;
        retire_block(c, b);
    }
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_cache_reset_counters(objeta_hip_expert_cache* c) {
    OBJ_TRY(check_cache(c, "cache reset_counters"));
    c->st.hit_count = c->st.miss_count = c->st.eviction_count = 0;
    c->st.cache_insert_attempt_count = c->st.cache_insert_accept_count = c->st.cache_insert_bypass_count = 0;
    c->st.oversized_tensor_bypass_count = c->st.oversized_expert_bypass_count = 0;
    c->st.self_eviction_risk_count = 0;
    return 0;
}

int32_t objeta_hip_cache_release_transient(objeta_hip_expert_cache* c, const void* d_ptr) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_cache(c, "release transient tensor"));
    auto it = c->transients.find(d_ptr);
    if (it == c->transients.end()) OBJ_FAIL(kInvalidInput, "release transient tensor", "unknown device pointer");
    Block* b = it->second;
    c->transients.erase(it);
    retire_block(c, b);
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_cache_prefetch(objeta_hip_expert_cache* c, const objeta_hip_cache_key* keys,
                                  const void* const* h_srcs, const uint64_t* nbytes, uint64_t n, uint64_t* issued) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_cache(c, "cache prefetch"));
    if (n && (!keys || !h_srcs || !nbytes)) OBJ_FAIL(kInvalidInput, "cache prefetch", "NULL argument");
    if (c->ctx) OBJ_HIP(hipSetDevice(c->ctx->device), "hipSetDevice");
    uint64_t done = 0;
    for (uint64_t i = 0; i < n; ++i) {
        const Key k = to_key(keys[i]);
        // resident keys and tensors the capacity could never hold are left alone
        if (c->map.count(k) || nbytes[i] > c->st.capacity_bytes) continue;
        Block* b = nullptr;
        OBJ_TRY(stage_tensor(c, h_srcs[i], nbytes[i], nullptr, &b));
        if (!insert_block(c, k, b, nbytes[i])) {
            retire_block(c, b);
            continue;
        }
        ++done;
    }
    if (issued) *issued = done;
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_cache_preload_shared(objeta_hip_expert_cache* c, const objeta_hip_host_expert* shared,
                                        uint64_t n_layers, uint64_t first_layer, objeta_hip_stream stream,
                                        uint64_t* bytes, float* ms) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_cache(c, "preload shared experts"));
    if (n_layers && !shared) OBJ_FAIL(kInvalidInput, "preload shared experts", "NULL shared expert array");
    const auto t0 = std::chrono::steady_clock::now();
    uint64_t total = 0;
    for (uint64_t l = 0; l < n_layers; ++l) {
        const objeta_hip_host_expert& e = shared[l];
        const struct {
            const void* h;
            uint64_t n;
            int32_t kind;
        } parts[6] = {{e.gate, e.gate_len, OBJETA_HIP_TENSOR_SHARED_GATE_WEIGHT},
                      {e.gate_scale, e.gate_scale_len, OBJETA_HIP_TENSOR_SHARED_GATE_SCALE},
                      {e.up, e.up_len, OBJETA_HIP_TENSOR_SHARED_UP_WEIGHT},
                      {e.up_scale, e.up_scale_len, OBJETA_HIP_TENSOR_SHARED_UP_SCALE},
                      {e.down, e.down_len, OBJETA_HIP_TENSOR_SHARED_DOWN_WEIGHT},
                      {e.down_scale, e.down_scale_len, OBJETA_HIP_TENSOR_SHARED_DOWN_SCALE}};
        for (const auto& p : parts) {
            objeta_hip_cache_key key{};
            key.layer_id = first_layer + l;
            key.expert_id = 0;
            key.tensor_kind = p.kind;
            key.quant_format = OBJETA_HIP_FP4_E2M1;
            const void* d = nullptr;
            OBJ_TRY(objeta_hip_cache_insert_pinned(c, &key, p.h, p.n, stream, &d));
            total += p.n;
        }
    }
    if (c->ctx && n_layers) OBJ_HIP(hipStreamSynchronize(c->ctx->copy_stream), "preload shared experts");
    if (bytes) *bytes = total;
    if (ms) *ms = std::chrono::duration<float, std::milli>(std::chrono::steady_clock::now() - t0).count();
    return 0;
    OBJ_GUARD_END
}

int32_t objeta_hip_cache_order(const objeta_hip_expert_cache* c, objeta_hip_cache_key* keys, uint64_t cap,
                               uint64_t* n) {
    OBJ_TRY(check_cache(c, "cache order"));
    if (!n) OBJ_FAIL(kInvalidInput, "cache order", "n is NULL");
    uint64_t i = 0;
    for (const Key& k : c->order) {
        if (keys && i < cap) keys[i] = from_key(k);
        ++i;
    }
    *n = i;
    return 0;
}

}  // extern "C"

// ------------------------------------------------------------------ executor
namespace objeta {
namespace {

struct TensorRef {
    const void* h;
    uint64_t len;
    int32_t kind;
    bool scale;
};

const char* tensor_label(int32_t kind) {
    switch (kind) {
        case OBJETA_HIP_TENSOR_GATE: return "w_gate";
        case OBJETA_HIP_TENSOR_UP: return "w_up";
        case OBJETA_HIP_TENSOR_DOWN: return "w_down";
        case OBJETA_HIP_TENSOR_GATE_WEIGHT: return "gate_weight";
        case OBJETA_HIP_TENSOR_GATE_SCALE: return "gate_scale";
        case OBJETA_HIP_TENSOR_UP_WEIGHT: return "up_weight";
        case OBJETA_HIP_TENSOR_UP_SCALE: return "up_scale";
        case OBJETA_HIP_TENSOR_DOWN_WEIGHT: return "down_weight";
        default: return "down_scale";
    }
}

// Per-context pool for transient (uncached) tensor copies; destroyed with the context.
Cache* transient_pool(objeta_hip_context* ctx) {
    if (!ctx->transient_pool) {
        Cache* c = new Cache();
        c->ctx = ctx;
        c->st.capacity_bytes = 0;
        ctx->transient_pool = c;
    }
    return static_cast<Cache*>(ctx->transient_pool);
}

float elapsed(hipEvent_t a, hipEvent_t b) {
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, a, b) != hipSuccess) {
        (void)hipGetLastError();
        return 0.f;
    }
    return ms;
}

// The tensors of one host expert in key order: w_gate / w_up / w_down for the
// block formats, gate/up/down weight and scale for the FP4 split layout.
int tensors_of(const objeta_hip_host_expert& e, bool fp4, TensorRef* t) {
    if (!fp4) {
        t[0] = {e.gate, e.gate_len, OBJETA_HIP_TENSOR_GATE, false};
        t[1] = {e.up, e.up_len, OBJETA_HIP_TENSOR_UP, false};
        t[2] = {e.down, e.down_len, OBJETA_HIP_TENSOR_DOWN, false};
        return 3;
    }
    t[0] = {e.gate, e.gate_len, OBJETA_HIP_TENSOR_GATE_WEIGHT, false};
    t[1] = {e.gate_scale, e.gate_scale_len, OBJETA_HIP_TENSOR_GATE_SCALE, true};
    t[2] = {e.up, e.up_len, OBJETA_HIP_TENSOR_UP_WEIGHT, false};
    t[3] = {e.up_scale, e.up_scale_len, OBJETA_HIP_TENSOR_UP_SCALE, true};
    t[4] = {e.down, e.down_len, OBJETA_HIP_TENSOR_DOWN_WEIGHT, false};
    t[5] = {e.down_scale, e.down_scale_len, OBJETA_HIP_TENSOR_DOWN_SCALE, true};
    return 6;
}

// The selected experts' device tensors for one executor call: cache hits, or
// copies of misses enqueued on the copy stream, with the byte accounting of the
// reference's load closure (moe.rs:458-583, 1000-1100, 1451-1487). The blocks stay
// referenced until release().
struct StagedExperts {
    std::vector<std::pair<Cache*, Block*>> held;  // (home, block) references of this call
    std::vector<hipEvent_t> ready;                // per slot: its copies done (NULL: all hits)
    uint64_t w_loaded = 0, w_reused = 0, s_loaded = 0, s_reused = 0, logical = 0;
    uint64_t by_kind[3] = {0, 0, 0};
    bool any_copy = false;

    Cache* events = nullptr;                      // where the ready events come from and go back
    hipStream_t stream = nullptr;                 // the call's stream, which reads the held blocks
    // Called once the call's kernels are enqueued: one mark on the call's stream ends
    // every held block's use by this call (so that a block evicted later needs no
    // fence once the mark has completed), then the references go.
    void release() {
        if (!held.empty() && stream && events) {
            const uint64_t id = mark_use(events, stream);
            for (auto& hb : held) set_last_use(hb.second, stream, id);
        }
        for (auto& hb : held) {
            hb.second->refs -= 1;
            retire_block(hb.first, hb.second);
        }
        held.clear();
    }
    ~StagedExperts() {
        for (hipEvent_t r : ready) {
            if (r && events) events->event_pool.push_back(r);
            else if (r) (void)hipEventDestroy(r);
        }
    }
};

// st.ready[j]: an event on the copy stream after slot j's copies.
int32_t record_ready(objeta_hip_context* ctx, Cache* pool, StagedExperts& st, uint64_t j) {
    hipEvent_t r = take_event(pool);
    if (!r || hipEventRecord(r, ctx->copy_stream) != hipSuccess) {
        (void)hipGetLastError();
        if (r) pool->event_pool.push_back(r);
        OBJ_FAIL(kDriver, "record copy event", "event failure");
    }
    st.ready[j] = r;
    return 0;
}

// count_oversize: an expert larger than the capacity counts as an oversized-expert
// bypass (bypass enabled) or a self-eviction risk, as the block-format and native
// FP4 executors count them (moe.rs:485-492); the official executor counts neither.
// batch: the pinned-source copies of all k experts go in one launch after the
// lookups, and one ready event after it stands for all of them (on the last slot with
// copies; for callers that wait for every slot before computing); else each copy is
// launched as its expert is staged and every slot with copies gets its own event.
int32_t stage_selected(objeta_hip_context* ctx, Cache* cache, const objeta_hip_host_expert* experts,
                       const uint64_t* sel_ids, uint64_t k, int32_t format, uint64_t layer_id, bool count_oversize,
                       hipStream_t s, objeta_hip_expert_ptrs* h_tab, StagedExperts& st, bool batch = false) {
    const bool fp4 = format == OBJETA_HIP_FP4_E2M1;
    Cache* pool = transient_pool(ctx);
    st.ready.assign(k, nullptr);
    st.events = pool;
    st.stream = s;
    // the copies are ordered after `s` once, at the first miss (each copy's own wait
    // would be one more stream wait per tensor)
    hipStream_t order_after = s;
    CopyBatch copies;
    std::vector<uint64_t> copied_slots;
    for (uint64_t j = 0; j < k; ++j) {
        const uint64_t e = sel_ids[j];
        TensorRef t[6];
        const int nt = tensors_of(experts[e], fp4, t);
        uint64_t eb = 0;
        for (int q = 0; q < nt; ++q) eb += t[q].len;
        st.logical += eb;
        st.by_kind[0] += t[0].len + (fp4 ? t[1].len : 0);
        st.by_kind[1] += fp4 ? t[2].len + t[3].len : t[1].len;
        st.by_kind[2] += fp4 ? t[4].len + t[5].len : t[2].len;
        bool bypass = false;
        if (cache && eb > cache->st.capacity_bytes) {
            if (cache->st.bypass_oversized_experts) {
                bypass = true;
                if (count_oversize) cache->st.oversized_expert_bypass_count += 1;
            } else if (count_oversize) {
                cache->st.self_eviction_risk_count += 1;
            }
        }
        const void* dptr[6] = {};
        bool copied = false;
        for (int q = 0; q < nt; ++q) {
            const Key key{layer_id, e, t[q].kind, format};
            Block* b = nullptr;
            bool hit = false;
            if (bypass) {
                cache->st.cache_insert_attempt_count += 1;
                cache->st.cache_insert_bypass_count += 1;
            } else if (cache) {
                b = lookup(cache, key);
                hit = b != nullptr;
                if (hit && cache->ctx) OBJ_TRY(wait_ready(cache, b, s));
            }
            Cache* home = cache && !bypass ? cache : pool;
            if (!hit) {
                const size_t pending = copies.blocks.size();
                OBJ_TRY(stage_tensor(home, t[q].h, t[q].len, order_after, &b, batch ? &copies : nullptr));
                order_after = nullptr;
                copied = true;
                const bool inserted = cache && !bypass && insert_block(cache, key, b, t[q].len);
                if (inserted && copies.blocks.size() > pending) {
                    copies.blocks.back().key = key;
                    copies.blocks.back().keyed = true;
                }
            }
            b->refs += 1;
            st.held.push_back({home, b});
            dptr[q] = b->ptr;
            if (hit) (t[q].scale ? st.s_reused : st.w_reused) += t[q].len;
            else (t[q].scale ? st.s_loaded : st.w_loaded) += t[q].len;
        }
        if (copied) {
            st.any_copy = true;
            copied_slots.push_back(j);
            if (!batch) OBJ_TRY(record_ready(ctx, pool, st, j));
        }
        objeta_hip_expert_ptrs& p = h_tab[j];
        if (fp4) p = {dptr[0], dptr[2], dptr[4], dptr[1], dptr[3], dptr[5]};
        else p = {dptr[0], dptr[1], dptr[2], nullptr, nullptr, nullptr};
    }
    if (batch) {
        OBJ_TRY(flush_copies(ctx, copies));
        // the one launch ends every copy of the call: one ready event, on the last slot
        // with copies, serves a caller that waits for all slots (one stream wait, not k)
        if (!copied_slots.empty()) OBJ_TRY(record_ready(ctx, pool, st, copied_slots.back()));
    }
    return 0;
}

// Size checks of every selected expert's tensors (moe.rs:366-422, 830-925).
int32_t validate_selected(const objeta_hip_host_expert* experts, uint64_t n_experts, const uint64_t* sel_ids,
                          uint64_t k, bool fp4, uint64_t gu_w, uint64_t gu_s, uint64_t dn_w, uint64_t dn_s) {
    for (uint64_t i = 0; i < k; ++i) {
        const uint64_t e = sel_ids[i];
        if (e >= n_experts)
            OBJ_FAIL(kInvalidInput, "validate expert index",
                     strf("expert index %llu out of bounds (len=%llu)", (unsigned long long)e,
                          (unsigned long long)n_experts));
        TensorRef t[6];
        const int nt = tensors_of(experts[e], fp4, t);
        for (int j = 0; j < nt; ++j) {
            const uint64_t want = (j < 2 * (nt / 3)) ? (t[j].scale ? gu_s : gu_w) : (t[j].scale ? dn_s : dn_w);
            if (t[j].len != want)
                OBJ_FAIL(kInvalidInput, strf("validate expert %s size", tensor_label(t[j].kind)),
                         strf("%s len %llu != expected %llu", tensor_label(t[j].kind), (unsigned long long)t[j].len,
                              (unsigned long long)want));
        }
    }
    return 0;
}

void copy_cache_counters(const Cache* cache, objeta_hip_moe_telemetry& t) {
    if (!cache) return;
    t.resident_cache_resident_bytes = cache->st.resident_bytes;
    t.resident_cache_capacity_bytes = cache->st.capacity_bytes;
    t.resident_cache_hit_count = cache->st.hit_count;
    t.resident_cache_miss_count = cache->st.miss_count;
    t.resident_cache_eviction_count = cache->st.eviction_count;
    t.resident_cache_insert_attempt_count = cache->st.cache_insert_attempt_count;
    t.resident_cache_insert_accept_count = cache->st.cache_insert_accept_count;
    t.resident_cache_insert_bypass_count = cache->st.cache_insert_bypass_count;
    t.resident_cache_oversized_tensor_bypass_count = cache->st.oversized_tensor_bypass_count;
    t.resident_cache_oversized_expert_bypass_count = cache->st.oversized_expert_bypass_count;
    t.resident_cache_self_eviction_risk_count = cache->st.self_eviction_risk_count;
}

struct EventSet {
    std::vector<hipEvent_t> e;
    explicit EventSet(size_t n) : e(n, nullptr) {}
    int32_t create() {
        for (auto& v : e) OBJ_HIP(hipEventCreate(&v), "create telemetry event");
        return 0;
    }
    ~EventSet() {
        for (hipEvent_t v : e)
            if (v) (void)hipEventDestroy(v);
    }
};

}  // namespace
}  // namespace objeta

extern "C" int32_t objeta_hip_moe_execute_selected(
    objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream, const objeta_hip_host_expert* experts,
    uint64_t n_experts, const uint64_t* sel_ids, const float* sel_weights, uint64_t n_selected, const float* x,
    uint64_t x_len, uint64_t hidden, uint64_t intermediate, uint64_t out_dim, uint64_t layer_id,
    objeta_hip_expert_cache* cache, float* out, objeta_hip_moe_telemetry* tel) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "execute_selected_moe"));
    const bool fp4 = format == OBJETA_HIP_FP4_E2M1;
    if (format < OBJETA_HIP_Q4_0 || format > OBJETA_HIP_FP4_E2M1)
        OBJ_FAIL(kUnsupported, "validate MoE format", strf("unsupported MoE format %d", format));
    if (cache && cache->ctx && cache->ctx != ctx)
        OBJ_FAIL(kInvalidInput, "validate expert cache", "cache belongs to another context");
    // ---- validation (moe.rs:366-422, 830-925)
    if (x_len != hidden)
        OBJ_FAIL(kInvalidInput,
                 fp4 ? "validate execute_selected_moe_native_fp4_cuda input x size"
                     : "validate execute_selected_moe_cuda input x size",
                 strf("x len %llu != hidden %llu", (unsigned long long)x_len, (unsigned long long)hidden));
    if (n_selected && (!sel_ids || !sel_weights)) OBJ_FAIL(kInvalidInput, "validate selection", "NULL selection");
    if ((hidden && !x) || (out_dim && !out)) OBJ_FAIL(kInvalidInput, "validate buffers", "NULL host pointer");
    const int32_t bb = objeta_hip_block_bytes(format);
    const uint64_t gu_w = fp4 ? intermediate * (hidden / 2) : intermediate * (hidden / 32) * bb;
    const uint64_t gu_s = fp4 ? intermediate * (hidden / 32) : 0;
    const uint64_t dn_w = fp4 ? out_dim * (intermediate / 2) : out_dim * (intermediate / 32) * bb;
    const uint64_t dn_s = fp4 ? out_dim * (intermediate / 32) : 0;
    OBJ_TRY(validate_selected(experts, n_experts, sel_ids, n_selected, fp4, gu_w, gu_s, dn_w, dn_s));
    if (n_selected > 32) OBJ_FAIL(kInvalidInput, "validate selection", "at most 32 selected experts per call");
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    hipStream_t s = resolve_stream(ctx, stream);
    const uint64_t k = n_selected;

    // ---- telemetry events
    enum { T0, X0, X1, GU0, GU1, DN1, D2H0, T1, C0, C1, kEv };
    EventSet evs(kEv);
    OBJ_TRY(evs.create());
    hipEvent_t* ev = evs.e.data();
    OBJ_HIP(hipEventRecord(ev[T0], s), "record event");

    // ---- device scratch: [x | out | weights | table] and host staging
    const size_t x_b = (hidden * 4 + 255) & ~size_t(255);
    const size_t o_b = (out_dim * 4 + 255) & ~size_t(255);
    const size_t w_b = 256;
    const size_t t_b = (k ? k : 1) * sizeof(objeta_hip_expert_ptrs);
    void* dws = nullptr;
    OBJ_TRY(ensure_workspace(ctx, s, kWsMoeTable, x_b + o_b + w_b + t_b, &dws));
    void* hst = nullptr;
    OBJ_TRY(ensure_host_stage(ctx, x_b + w_b + t_b + o_b, &hst));
    char* d0 = static_cast<char*>(dws);
    float* d_x = reinterpret_cast<float*>(d0);
    float* d_out = reinterpret_cast<float*>(d0 + x_b);
    float* d_w = reinterpret_cast<float*>(d0 + x_b + o_b);
    objeta_hip_expert_ptrs* d_tab = reinterpret_cast<objeta_hip_expert_ptrs*>(d0 + x_b + o_b + w_b);
    char* h0 = static_cast<char*>(hst);
    std::memcpy(h0, x, hidden * 4);
    if (k) std::memcpy(h0 + x_b + o_b, sel_weights, k * 4);
    objeta_hip_expert_ptrs* h_tab = reinterpret_cast<objeta_hip_expert_ptrs*>(h0 + x_b + o_b + w_b);
    float* h_out = reinterpret_cast<float*>(h0 + x_b);
    OBJ_HIP(hipEventRecord(ev[X0], s), "record event");
    OBJ_HIP(hipMemcpyAsync(d_x, h0, hidden * 4, hipMemcpyHostToDevice, s), "moe_x_h2d");
    OBJ_HIP(hipEventRecord(ev[X1], s), "record event");

    // ---- weights: cache admission and copies (moe.rs:458-583, 1000-1100)
    StagedExperts st;
    OBJ_HIP(hipEventRecord(ev[C0], ctx->copy_stream), "record event");
    std::vector<uint64_t> uniq(sel_ids, sel_ids + k);
    std::sort(uniq.begin(), uniq.end());
    uniq.erase(std::unique(uniq.begin(), uniq.end()), uniq.end());
    const uint64_t single_expert_bytes = 2 * (gu_w + gu_s) + dn_w + dn_s;
    int32_t rc = stage_selected(ctx, cache, experts, sel_ids, k, format, layer_id, true, s, h_tab, st);
    if (rc) {
        (void)hipStreamSynchronize(ctx->copy_stream);
        st.release();
        return rc;
    }
    OBJ_HIP(hipEventRecord(ev[C1], ctx->copy_stream), "record event");

    // ---- compute
    do {
        if (k) {
            hipError_t e = hipMemcpyAsync(d_w, h0 + x_b + o_b, w_b + t_b, hipMemcpyHostToDevice, s);
            if (e != hipSuccess) {
                (void)hipGetLastError();
                rc = set_error(kDriver, __FILE__, __LINE__, __func__, "moe_table_h2d", hipGetErrorString(e));
                break;
            }
        }
        float* act = nullptr;
        if ((rc = moe_act_scratch(ctx, s, 1, k ? k : 1, intermediate ? intermediate : 1, &act))) break;
        (void)hipEventRecord(ev[GU0], s);
        if (k == 0) {
            if ((rc = launch_zero(s, d_out, out_dim * 4))) break;
            (void)hipEventRecord(ev[GU1], s);
        } else if (!st.any_copy) {
            if ((rc = launch_moe_gate_up(ctx, format, s, d_tab, k, nullptr, 1, k, d_x, act, hidden, intermediate, 0.f)))
                break;
            (void)hipEventRecord(ev[GU1], s);
            if ((rc = launch_moe_down(ctx, format, s, d_tab, k, nullptr, d_w, 1, k, act, nullptr, d_out, intermediate,
                                      out_dim)))
                break;
        } else {
            // expert by expert, each waiting only for its own copies
            for (uint64_t j = 0; j < k && rc == 0; ++j) {
                if (st.ready[j]) {
                    hipError_t e = hipStreamWaitEvent(s, st.ready[j], 0);
                    if (e != hipSuccess) {
                        (void)hipGetLastError();
                        rc = set_error(kDriver, __FILE__, __LINE__, __func__, "wait expert copies", hipGetErrorString(e));
                        break;
                    }
                }
                rc = launch_moe_gate_up(ctx, format, s, d_tab + j, 1, nullptr, 1, 1, d_x, act, hidden, intermediate, 0.f);
                if (!rc)
                    rc = launch_moe_down(ctx, format, s, d_tab + j, 1, nullptr, d_w + j, 1, 1, act, j ? d_out : nullptr,
                                         d_out, intermediate, out_dim);
            }
            (void)hipEventRecord(ev[GU1], s);
        }
        if (rc) break;
        (void)hipEventRecord(ev[DN1], s);
        (void)hipEventRecord(ev[D2H0], s);
        hipError_t e = hipMemcpyAsync(h_out, d_out, out_dim * 4, hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipEventRecord(ev[T1], s);
        if (e == hipSuccess) e = hipEventSynchronize(ev[T1]);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            rc = set_error(kDriver, __FILE__, __LINE__, __func__, "moe_d2h", hipGetErrorString(e));
        }
    } while (false);
    if (rc) {
        (void)hipStreamSynchronize(s);
        (void)hipStreamSynchronize(ctx->copy_stream);
        st.release();
        return rc;
    }
    std::memcpy(out, h_out, out_dim * 4);
    st.release();

    // ---- telemetry (moe.rs:664-748)
    const uint64_t loaded = st.w_loaded + st.s_loaded, reused = st.w_reused + st.s_reused;
    if (st.logical != loaded + reused)
        OBJ_FAIL(kInternal, "MoE byte invariant", "logical_expert_bytes_requested != loaded + reused");
    if (tel) {
        objeta_hip_moe_telemetry t{};
        t.selected_expert_count = k;
        t.logical_expert_bytes_requested = st.logical;
        t.actual_expert_bytes_loaded = loaded;
        t.resident_cache_bytes_reused = reused;
        t.weight_bytes_loaded = st.w_loaded;
        t.weight_bytes_reused = st.w_reused;
        t.scale_bytes_loaded = st.s_loaded;
        t.scale_bytes_reused = st.s_reused;
        copy_cache_counters(cache, t);
        t.h2d_ms = elapsed(ev[X0], ev[X1]) + (st.any_copy ? elapsed(ev[C0], ev[C1]) : 0.f);
        t.gate_up_qgemv_ms = elapsed(ev[GU0], ev[GU1]);
        t.down_qgemv_ms = elapsed(ev[GU1], ev[DN1]);
        const float d2h = elapsed(ev[D2H0], ev[T1]);
        t.total_ms = elapsed(ev[T0], ev[T1]);
        const float un = t.total_ms - t.h2d_ms - t.gate_up_qgemv_ms - t.down_qgemv_ms - d2h;
        t.unaccounted_ms = un > 0.f ? un : 0.f;
        t.bytes_by_tensor_kind_gate = st.by_kind[0];
        t.bytes_by_tensor_kind_up = st.by_kind[1];
        t.bytes_by_tensor_kind_down = st.by_kind[2];
        t.bytes_per_expert = single_expert_bytes;
        t.selected_working_set_bytes = uniq.size() * single_expert_bytes;
        *tel = t;
    }
    return 0;
    OBJ_GUARD_END
}

// execute_selected_moe_official_routed_fp4_cuda (moe.rs:1393-1663): FP4 split
// routed experts through the FP8-activation path, plus an optional device-resident
// FP8 shared expert, for one token. The launches are those of
// objeta_hip_moe_official_fp4_device; misses are copied on the copy stream and the
// layer waits for all of them. Telemetry follows the reference's official
// accounting: logical bytes are the unique selected experts' working set, the
// shared expert counts as loaded on every call, cache counters beyond
// hit/miss/eviction stay 0, activation_ms is the intermediate act_quant and
// shared_expert_ms the shared expert's two launches.
extern "C" int32_t objeta_hip_moe_execute_official_fp4(
    objeta_hip_context* ctx, objeta_hip_stream stream, const objeta_hip_host_expert* experts, uint64_t n_experts,
    const uint64_t* sel_ids, const float* sel_weights, uint64_t n_selected, const float* x, uint64_t x_len,
    uint64_t hidden, uint64_t intermediate, uint64_t out_dim, uint64_t layer_id, objeta_hip_expert_cache* cache,
    const objeta_hip_expert_ptrs* shared_fp8, int32_t shared_from_cache, float swiglu_limit, float* out,
    objeta_hip_moe_telemetry* tel) {
    OBJ_GUARD_BEGIN
    OBJ_TRY(check_ctx(ctx, "execute_selected_moe_official_routed_fp4"));
    const char* action = "validate execute_selected_moe_official_routed_fp4_cuda input";
    if (cache && cache->ctx && cache->ctx != ctx)
        OBJ_FAIL(kInvalidInput, "validate expert cache", "cache belongs to another context");
    if (x_len != hidden)
        OBJ_FAIL(kInvalidInput, action,
                 strf("x len %llu != hidden %llu", (unsigned long long)x_len, (unsigned long long)hidden));
    if (hidden % 128 != 0 || intermediate % 128 != 0)
        OBJ_FAIL(kInvalidInput, action,
                 strf("hidden %llu and intermediate %llu must be multiples of 128", (unsigned long long)hidden,
                      (unsigned long long)intermediate));
    if (n_selected && (!sel_ids || !sel_weights)) OBJ_FAIL(kInvalidInput, "validate selection", "NULL selection");
    if ((hidden && !x) || (out_dim && !out)) OBJ_FAIL(kInvalidInput, "validate buffers", "NULL host pointer");
    const uint64_t gu_w = intermediate * (hidden / 2), gu_s = intermediate * (hidden / 32);
    const uint64_t dn_w = out_dim * (intermediate / 2), dn_s = out_dim * (intermediate / 32);
    OBJ_TRY(validate_selected(experts, n_experts, sel_ids, n_selected, true, gu_w, gu_s, dn_w, dn_s));
    if (n_selected > 32) OBJ_FAIL(kInvalidInput, "validate selection", "at most 32 selected experts per call");
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    hipStream_t s = resolve_stream(ctx, stream);
    const uint64_t k = n_selected;

    enum { T0, X0, X1, GU1, SH1, AQ1, DN1, D2H0, T1, kEv };
    EventSet evs(kEv);
    OBJ_TRY(evs.create());
    hipEvent_t* ev = evs.e.data();
    OBJ_HIP(hipEventRecord(ev[T0], s), "record event");

    // device scratch: [x | out | weights | ids | table | shared entry] and host staging
    const size_t x_b = (hidden * 4 + 255) & ~size_t(255);
    const size_t o_b = (out_dim * 4 + 255) & ~size_t(255);
    const size_t w_b = 256, i_b = 256;
    const size_t t_b = (k + 1) * sizeof(objeta_hip_expert_ptrs);
    void* dws = nullptr;
    OBJ_TRY(ensure_workspace(ctx, s, kWsMoeTable, x_b + o_b + w_b + i_b + t_b, &dws));
    void* hst = nullptr;
    OBJ_TRY(ensure_host_stage(ctx, x_b + o_b + w_b + i_b + t_b, &hst));
    char* d0 = static_cast<char*>(dws);
    char* h0 = static_cast<char*>(hst);
    float* d_x = reinterpret_cast<float*>(d0);
    float* d_out = reinterpret_cast<float*>(d0 + x_b);
    float* h_out = reinterpret_cast<float*>(h0 + x_b);
    const size_t tail = x_b + o_b;  // weights | ids | table, copied in one piece
    float* d_w = reinterpret_cast<float*>(d0 + tail);
    uint32_t* d_ids = reinterpret_cast<uint32_t*>(d0 + tail + w_b);
    objeta_hip_expert_ptrs* d_tab = reinterpret_cast<objeta_hip_expert_ptrs*>(d0 + tail + w_b + i_b);
    uint32_t* h_ids = reinterpret_cast<uint32_t*>(h0 + tail + w_b);
    objeta_hip_expert_ptrs* h_tab = reinterpret_cast<objeta_hip_expert_ptrs*>(h0 + tail + w_b + i_b);
    std::memcpy(h0, x, hidden * 4);
    if (k) std::memcpy(h0 + tail, sel_weights, k * 4);
    for (uint64_t j = 0; j < k; ++j) h_ids[j] = static_cast<uint32_t>(j);  // slot j reads table entry j
    OBJ_HIP(hipEventRecord(ev[X0], s), "record event");
    OBJ_HIP(hipMemcpyAsync(d_x, h0, hidden * 4, hipMemcpyHostToDevice, s), "official_h2d");
    OBJ_HIP(hipEventRecord(ev[X1], s), "record event");

    StagedExperts st;
    int32_t rc =
        stage_selected(ctx, cache, experts, sel_ids, k, OBJETA_HIP_FP4_E2M1, layer_id, false, s, h_tab, st, true);
    // The shared expert: with shared_from_cache, the cache's six Shared* entries of
    // this layer first (get in key order, stopping at the first miss, as the sketch
    // in crates/objeta-cuda/src/moe_tmp.txt:1-35 resolves it), else the argument.
    bool have_sh = false, sh_cached = false;
    uint64_t sh_cached_bytes = 0;
    if (rc == 0 && shared_from_cache && cache) {
        const int32_t kinds[6] = {OBJETA_HIP_TENSOR_SHARED_GATE_WEIGHT, OBJETA_HIP_TENSOR_SHARED_GATE_SCALE,
                                  OBJETA_HIP_TENSOR_SHARED_UP_WEIGHT,   OBJETA_HIP_TENSOR_SHARED_UP_SCALE,
                                  OBJETA_HIP_TENSOR_SHARED_DOWN_WEIGHT, OBJETA_HIP_TENSOR_SHARED_DOWN_SCALE};
        const void* p[6] = {};
        uint64_t sz[6] = {};
        int q = 0;
        for (; q < 6 && rc == 0; ++q) {
            const Key key{layer_id, 0, kinds[q], OBJETA_HIP_FP4_E2M1};
            Block* b = lookup(cache, key);
            if (!b) break;
            if (cache->ctx) rc = wait_ready(cache, b, s);
            b->refs += 1;
            st.held.push_back({cache, b});
            p[q] = b->ptr;
            sz[q] = cache->map.find(key)->second.size;
            sh_cached_bytes += sz[q];
        }
        if (rc == 0 && q == 6) {
            // the FP8 shared expert of this shape: E4M3 codes [rows][cols] and E8M0
            // scales on the 128 x 128 tile grid; entries preloaded for another shape
            // would be read past their ends
            const uint64_t ti = (intermediate + 127) / 128, th = (hidden + 127) / 128, to = (out_dim + 127) / 128;
            const uint64_t want[6] = {intermediate * hidden, ti * th, intermediate * hidden, ti * th,
                                      out_dim * intermediate, to * ti};
            const char* names[6] = {"gate weight", "gate scale", "up weight", "up scale", "down weight", "down scale"};
            for (int i = 0; i < 6 && rc == 0; ++i)
                if (sz[i] != want[i])
                    rc = set_error(kInvalidInput, __FILE__, __LINE__, __func__, "resolve cached shared expert",
                                   strf("layer %llu shared %s holds %llu bytes, expected %llu for hidden %llu, "
                                        "intermediate %llu, out_dim %llu",
                                        (unsigned long long)layer_id, names[i], (unsigned long long)sz[i],
                                        (unsigned long long)want[i], (unsigned long long)hidden,
                                        (unsigned long long)intermediate, (unsigned long long)out_dim));
        }
        if (rc == 0 && q == 6) {
            h_tab[k] = {p[0], p[2], p[4], p[1], p[3], p[5]};
            have_sh = sh_cached = true;
        }
    }
    if (!have_sh && shared_fp8) {
        h_tab[k] = *shared_fp8;
        have_sh = true;
    }
    if (rc) {
        (void)hipStreamSynchronize(ctx->copy_stream);
        st.release();
        return rc;
    }
    do {
        hipError_t e = hipMemcpyAsync(d0 + tail, h0 + tail, w_b + i_b + t_b, hipMemcpyHostToDevice, s);
        for (uint64_t j = 0; j < k && e == hipSuccess; ++j)
            if (st.ready[j]) e = hipStreamWaitEvent(s, st.ready[j], 0);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            rc = set_error(kDriver, __FILE__, __LINE__, __func__, "official_table_h2d", hipGetErrorString(e));
            break;
        }
        const OfficialMarks marks{ev[GU1], ev[SH1], ev[AQ1], ev[DN1]};
        if ((rc = launch_moe_official_fp4(ctx, s, d_tab, k ? k : 1, have_sh ? d_tab + k : nullptr, d_ids, d_w, 1, k,
                                          d_x, d_out, hidden, intermediate, out_dim, swiglu_limit, nullptr, nullptr,
                                          &marks)))
            break;
        (void)hipEventRecord(ev[D2H0], s);
        e = hipMemcpyAsync(h_out, d_out, out_dim * 4, hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipEventRecord(ev[T1], s);
        if (e == hipSuccess) e = hipEventSynchronize(ev[T1]);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            rc = set_error(kDriver, __FILE__, __LINE__, __func__, "official_d2h", hipGetErrorString(e));
        }
    } while (false);
    if (rc) {
        (void)hipStreamSynchronize(s);
        (void)hipStreamSynchronize(ctx->copy_stream);
        st.release();
        return rc;
    }
    std::memcpy(out, h_out, out_dim * 4);
    st.release();

    if (tel) {
        std::vector<uint64_t> uniq(sel_ids, sel_ids + k);
        std::sort(uniq.begin(), uniq.end());
        uniq.erase(std::unique(uniq.begin(), uniq.end()), uniq.end());
        const uint64_t single_expert_bytes = 2 * (gu_w + gu_s) + dn_w + dn_s;
        const uint64_t working = uniq.size() * single_expert_bytes;
        // the reference's shared byte formula (moe.rs:1618-1624), scales counted per 128;
        // a shared expert taken from the cache counts its resident bytes as reused
        const uint64_t sh_formula = 2 * (intermediate * hidden) + out_dim * intermediate +
                                    2 * (intermediate * hidden / 128) + out_dim * intermediate / 128;
        const uint64_t sh_total = sh_cached ? sh_cached_bytes : (have_sh ? sh_formula : 0);
        const uint64_t sh_loaded = sh_cached ? 0 : sh_total;
        const uint64_t loaded = st.w_loaded + st.s_loaded, reused = st.w_reused + st.s_reused;
        objeta_hip_moe_telemetry t{};
        t.selected_expert_count = k;
        t.logical_expert_bytes_requested = working;
        t.actual_expert_bytes_loaded = loaded;
        t.resident_cache_bytes_reused = reused;
        t.weight_bytes_loaded = st.w_loaded;
        t.weight_bytes_reused = st.w_reused;
        t.scale_bytes_loaded = st.s_loaded;
        t.scale_bytes_reused = st.s_reused;
        if (cache) {
            t.resident_cache_resident_bytes = cache->st.resident_bytes;
            t.resident_cache_capacity_bytes = cache->st.capacity_bytes;
            t.resident_cache_hit_count = cache->st.hit_count;
            t.resident_cache_miss_count = cache->st.miss_count;
            t.resident_cache_eviction_count = cache->st.eviction_count;
        }
        t.h2d_ms = elapsed(ev[X0], ev[X1]);
        t.gate_up_qgemv_ms = elapsed(ev[X1], ev[GU1]);
        t.activation_ms = elapsed(ev[SH1], ev[AQ1]);
        t.down_qgemv_ms = elapsed(ev[AQ1], ev[DN1]);
        t.shared_expert_ms = have_sh ? elapsed(ev[GU1], ev[SH1]) + elapsed(ev[DN1], ev[D2H0]) : 0.f;
        t.total_ms = elapsed(ev[T0], ev[T1]) - elapsed(ev[D2H0], ev[T1]);
        t.bytes_per_expert = single_expert_bytes;
        t.selected_working_set_bytes = working;
        t.routed_fp4_bytes_loaded = loaded;
        t.routed_fp4_bytes_reused = reused;
        t.shared_fp8_bytes_loaded = sh_loaded;
        t.shared_fp8_bytes_reused = sh_total - sh_loaded;
        t.total_logical_bytes = working + sh_total;
        t.total_loaded_bytes = loaded + sh_loaded;
        t.total_reused_bytes = reused + (sh_total - sh_loaded);
        *tel = t;
    }
    return 0;
    OBJ_GUARD_END
}

// ------------------------------------------------------------ cached decode stack
// The loop the reference's drivers run over execute_selected_moe_cuda, with the
// hidden state on the device: per layer one host wait (the router's ids), the
// union of the batch's experts resolved through the cache, the layer's kernels
// behind its own copies. Scratch (device and pinned host, one layout):
// [ids | weights | predicted ids | predicted weights | remapped ids | table].
extern "C" int32_t objeta_hip_moe_stack_cached(objeta_hip_context* ctx, int32_t format, objeta_hip_stream stream,
                                               const objeta_hip_cached_layer* layers, uint64_t n_layers, uint64_t k,
                                               int32_t renormalize, uint64_t n_tokens, float* d_h, uint64_t hidden,
                                               uint64_t intermediate, objeta_hip_expert_cache* cache,
                                               int32_t prefetch_next, uint32_t* ids_out, float* weights_out,
                                               float* d_trace, objeta_hip_stack_telemetry* tel) {
    OBJ_GUARD_BEGIN
    using namespace objeta;
    const char* action = "moe_stack_cached";
    OBJ_TRY(check_ctx(ctx, action));
    if (format < OBJETA_HIP_Q4_0 || format > OBJETA_HIP_FP4_E2M1)
        OBJ_FAIL(kUnsupported, action, strf("unsupported MoE format %d", format));
    if (cache && cache->ctx && cache->ctx != ctx) OBJ_FAIL(kInvalidInput, action, "cache belongs to another context");
    if (tel) *tel = objeta_hip_stack_telemetry{};
    if (n_layers == 0 || n_tokens == 0) return 0;
    if (!layers || !d_h) OBJ_FAIL(kInvalidInput, action, "NULL layers or hidden state");
    if (k == 0 || k > 32) OBJ_FAIL(kInvalidInput, action, strf("k %llu must be in 1..=32", (unsigned long long)k));
    if (n_tokens > 256) OBJ_FAIL(kInvalidInput, action, "at most 256 tokens per call");
    if (hidden == 0 || intermediate == 0 || hidden % 32 || intermediate % 32)
        OBJ_FAIL(kInvalidInput, action,
                 strf("hidden %llu and intermediate %llu must be non-zero multiples of block_size 32",
                      (unsigned long long)hidden, (unsigned long long)intermediate));
    const bool fp4 = format == OBJETA_HIP_FP4_E2M1;
    const int32_t bb = objeta_hip_block_bytes(format);
    const uint64_t gu_w = fp4 ? intermediate * (hidden / 2) : intermediate * (hidden / 32) * bb;
    const uint64_t gu_s = fp4 ? intermediate * (hidden / 32) : 0;
    const uint64_t dn_w = fp4 ? hidden * (intermediate / 2) : hidden * (intermediate / 32) * bb;
    const uint64_t dn_s = fp4 ? hidden * (intermediate / 32) : 0;
    // every layer's experts against the shape, before anything is enqueued
    for (uint64_t l = 0; l < n_layers; ++l) {
        const objeta_hip_cached_layer& L = layers[l];
        if (!L.experts || !L.d_router_w)
            OBJ_FAIL(kInvalidInput, action, strf("layer %llu: NULL experts or router", (unsigned long long)l));
        if (L.n_experts < k)
            OBJ_FAIL(kInvalidInput, action,
                     strf("layer %llu: %llu experts for top-%llu", (unsigned long long)l,
                          (unsigned long long)L.n_experts, (unsigned long long)k));
        std::vector<uint64_t> all(L.n_experts);
        for (uint64_t e = 0; e < L.n_experts; ++e) all[e] = e;
        OBJ_TRY(validate_selected(L.experts, L.n_experts, all.data(), L.n_experts, fp4, gu_w, gu_s, dn_w, dn_s));
    }
    OBJ_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    hipStream_t s = resolve_stream(ctx, stream);
    const uint64_t T = n_tokens, tk = n_tokens * k;
    auto up = [](size_t v) { return (v + 255) & ~size_t(255); };
    const size_t o_ids = 0, o_w = up(tk * 4), o_pids = o_w + up(tk * 4), o_pw = o_pids + up(tk * 4);
    const size_t o_rids = o_pw + up(tk * 4), o_tab = o_rids + up(tk * 4);
    const size_t total = o_tab + tk * sizeof(objeta_hip_expert_ptrs);
    void* dws = nullptr;
    OBJ_TRY(ensure_workspace(ctx, s, kWsStack, total, &dws));
    void* hst = nullptr;
    OBJ_TRY(ensure_host_stage(ctx, total, &hst));
    char* d0 = static_cast<char*>(dws);
    char* h0 = static_cast<char*>(hst);
    uint32_t* d_ids = reinterpret_cast<uint32_t*>(d0 + o_ids);
    float* d_w = reinterpret_cast<float*>(d0 + o_w);
    uint32_t* d_pids = reinterpret_cast<uint32_t*>(d0 + o_pids);
    float* d_pw = reinterpret_cast<float*>(d0 + o_pw);
    const uint32_t* d_rids = reinterpret_cast<const uint32_t*>(d0 + o_rids);
    const objeta_hip_expert_ptrs* d_tab = reinterpret_cast<const objeta_hip_expert_ptrs*>(d0 + o_tab);
    const uint32_t* h_ids = reinterpret_cast<const uint32_t*>(h0 + o_ids);
    const float* h_w = reinterpret_cast<const float*>(h0 + o_w);
    const uint32_t* h_pids = reinterpret_cast<const uint32_t*>(h0 + o_pids);
    uint32_t* h_rids = reinterpret_cast<uint32_t*>(h0 + o_rids);
    objeta_hip_expert_ptrs* h_tab = reinterpret_cast<objeta_hip_expert_ptrs*>(h0 + o_tab);

    const size_t ev_t0 = 0, ev_t1 = 1, ev_route = 2, ev_c = 3;  // then (c0, c1) per layer
    EventSet evs(3 + 2 * n_layers);
    OBJ_TRY(evs.create());
    hipEvent_t* ev = evs.e.data();
    objeta_hip_stack_telemetry t{};
    t.layers = n_layers;
    t.tokens = T;
    double wait_ms = 0.0;
    std::vector<uint32_t> predicted;  // this layer's experts as the previous layer predicted them
    std::vector<uint64_t> uni;
    std::vector<char> seen;
    OBJ_HIP(hipEventRecord(ev[ev_t0], s), "record event");
    for (uint64_t l = 0; l < n_layers; ++l) {
        const objeta_hip_cached_layer& L = layers[l];
        const bool pf = prefetch_next && cache && cache->ctx && l + 1 < n_layers;
        // ---- routing: this layer's router, and the next layer's on the same input
        OBJ_TRY(launch_router(ctx, s, L.d_router_w, L.d_router_bias, d_h, T, L.n_experts, hidden, k, renormalize,
                              d_ids, d_w, nullptr, nullptr));
        if (pf) {
            const objeta_hip_cached_layer& N = layers[l + 1];
            OBJ_TRY(launch_router(ctx, s, N.d_router_w, N.d_router_bias, d_h, T, N.n_experts, hidden, k, renormalize,
                                  d_pids, d_pw, nullptr, nullptr));
        }
        OBJ_HIP(hipMemcpyAsync(h0, d0, pf ? o_rids : o_pids, hipMemcpyDeviceToHost, s), "stack_ids_d2h");
        OBJ_HIP(hipEventRecord(ev[ev_route], s), "record event");
        const auto w0 = std::chrono::steady_clock::now();
        OBJ_HIP(hipEventSynchronize(ev[ev_route]), "wait for the router");
        wait_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - w0).count();
        for (uint64_t i = 0; i < tk; ++i)
            if (h_ids[i] >= L.n_experts)
                OBJ_FAIL(kInternal, action, strf("router id %u out of range at layer %llu", h_ids[i],
                                                 (unsigned long long)l));
        if (ids_out) std::memcpy(ids_out + l * tk, h_ids, tk * 4);
        if (weights_out) std::memcpy(weights_out + l * tk, h_w, tk * 4);
        if (!predicted.empty()) {  // the previous layer's prediction of these selections, per token
            for (uint64_t tt = 0; tt < T; ++tt)
                for (uint64_t a = 0; a < k; ++a)
                    for (uint64_t b = 0; b < k; ++b)
                        if (predicted[tt * k + a] == h_ids[tt * k + b]) {
                            t.prefetch_experts_correct += 1;
                            break;
                        }
            t.prefetch_experts_predicted += tk;
        }
        // ---- the union of the batch's experts through the cache
        uni.assign(h_ids, h_ids + tk);
        std::sort(uni.begin(), uni.end());
        uni.erase(std::unique(uni.begin(), uni.end()), uni.end());
        for (uint64_t i = 0; i < tk; ++i)
            h_rids[i] = static_cast<uint32_t>(std::lower_bound(uni.begin(), uni.end(), h_ids[i]) - uni.begin());
        hipEvent_t c0 = ev[ev_c + 2 * l], c1 = ev[ev_c + 2 * l + 1];
        OBJ_HIP(hipEventRecord(c0, ctx->copy_stream), "record event");
        StagedExperts st;
        int32_t rc = stage_selected(ctx, cache, L.experts, uni.data(), uni.size(), format, L.layer_id, true, s, h_tab,
                                    st, true);
        if (rc == 0 && hipEventRecord(c1, ctx->copy_stream) != hipSuccess) {
            (void)hipGetLastError();
            rc = set_error(kDriver, __FILE__, __LINE__, __func__, "record event", "copy-stream event failed");
        }
        // ---- the next layer's predicted experts, copied behind this layer's misses
        if (rc == 0 && pf) {
            const objeta_hip_cached_layer& N = layers[l + 1];
            predicted.assign(h_pids, h_pids + tk);
            seen.assign(N.n_experts, 0);
            CopyBatch pf_copies;  // the predictions' copies, in one launch after the lookups
            for (uint64_t i = 0; i < tk && rc == 0; ++i) {
                const uint32_t p = h_pids[i];
                if (p >= N.n_experts || seen[p]) continue;
                seen[p] = 1;
                TensorRef tr[6];
                const int nt = tensors_of(N.experts[p], fp4, tr);
                for (int q = 0; q < nt && rc == 0; ++q) {
                    const Key key{N.layer_id, p, tr[q].kind, format};
                    if (cache->map.count(key) || tr[q].len > cache->st.capacity_bytes) continue;
                    Block* b = nullptr;
                    const size_t pending = pf_copies.blocks.size();
                    if ((rc = stage_tensor(cache, tr[q].h, tr[q].len, nullptr, &b, &pf_copies))) break;
                    (void)insert_block(cache, key, b, tr[q].len);  // fits: larger tensors were skipped
                    if (pf_copies.blocks.size() > pending) {
                        pf_copies.blocks.back().key = key;
                        pf_copies.blocks.back().keyed = true;
                    }
                    t.prefetch_tensors_issued += 1;
                    t.prefetch_bytes_issued += tr[q].len;
                }
            }
            if (rc == 0) rc = flush_copies(ctx, pf_copies);
        } else {
            predicted.clear();
        }
        // ---- the layer, after its own copies
        do {
            if (rc) break;
            // the remapped ids and the table (from the pinned host stage, by a kernel when it can)
            const size_t tb = (o_tab - o_rids) + uni.size() * sizeof(objeta_hip_expert_ptrs);
            const void* hs = pinned_device_ptr(h0 + o_rids, tb);
            hipError_t e = hipSuccess;
            if (hs) {
                if ((rc = launch_h2d_copy(s, d0 + o_rids, hs, tb))) break;
            } else {
                e = hipMemcpyAsync(d0 + o_rids, h0 + o_rids, tb, hipMemcpyHostToDevice, s);
            }
            for (size_t j = 0; j < uni.size() && e == hipSuccess; ++j)
                if (st.ready[j]) e = hipStreamWaitEvent(s, st.ready[j], 0);
            if (e != hipSuccess) {
                (void)hipGetLastError();
                rc = set_error(kDriver, __FILE__, __LINE__, __func__, "stack_table_h2d", hipGetErrorString(e));
                break;
            }
            if (grouped_preferred(format, T, hidden, intermediate, hidden) &&
                grouped_supported(format, uni.size(), T, k, hidden, intermediate, hidden)) {
                rc = launch_moe_grouped(ctx, format, s, d_tab, uni.size(), nullptr, d_rids, d_w, T, k, d_h, d_h, d_h,
                                        hidden, intermediate, hidden, 0.f);
            } else {
                float* act = nullptr;
                if ((rc = moe_act_scratch(ctx, s, T, k, intermediate, &act))) break;
                rc = launch_moe_gate_up(ctx, format, s, d_tab, uni.size(), d_rids, T, k, d_h, act, hidden,
                                        intermediate, 0.f);
                if (!rc)
                    rc = launch_moe_down(ctx, format, s, d_tab, uni.size(), d_rids, d_w, T, k, act, d_h, d_h,
                                         intermediate, hidden);
            }
            if (rc == 0 && d_trace) {
                e = hipMemcpyAsync(d_trace + l * T * hidden, d_h, T * hidden * 4, hipMemcpyDeviceToDevice, s);
                if (e != hipSuccess) {
                    (void)hipGetLastError();
                    rc = set_error(kDriver, __FILE__, __LINE__, __func__, "stack_trace_d2d", hipGetErrorString(e));
                }
            }
        } while (false);
        // the blocks stay valid for the kernels enqueued above: a block evicted from
        // now on is fenced behind them before it is reused
        st.release();
        if (rc) {
            (void)hipStreamSynchronize(s);
            (void)hipStreamSynchronize(ctx->copy_stream);
            return rc;
        }
        t.logical_expert_bytes_requested += st.logical;
        t.actual_expert_bytes_loaded += st.w_loaded + st.s_loaded;
        t.resident_cache_bytes_reused += st.w_reused + st.s_reused;
        t.distinct_experts += uni.size();
    }
    OBJ_HIP(hipEventRecord(ev[ev_t1], s), "record event");
    OBJ_HIP(hipEventSynchronize(ev[ev_t1]), "wait for the stack");
    if (t.logical_expert_bytes_requested != t.actual_expert_bytes_loaded + t.resident_cache_bytes_reused)
        OBJ_FAIL(kInternal, "MoE byte invariant", "logical_expert_bytes_requested != loaded + reused");
    t.total_ms = elapsed(ev[ev_t0], ev[ev_t1]);
    for (uint64_t l = 0; l < n_layers; ++l) t.copy_ms += elapsed(ev[ev_c + 2 * l], ev[ev_c + 2 * l + 1]);
    t.host_wait_ms = static_cast<float>(wait_ms);
    if (tel) *tel = t;
    return 0;
    OBJ_GUARD_END
}
