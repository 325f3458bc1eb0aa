// Blob (mmap + manifest + layout check) and the 2-slot host ring with its
// reader thread — ltx/loader.zig:45-92 and :176-321 over the same format.
// Slot states free -> filling -> ready -> in_use -> free are asserted on every
// transition; an illegal move aborts the process, as the reference panics.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <chrono>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <mutex>
#include <sstream>
#include <string>
#include <thread>
#include <vector>

#include "json.hpp"
#include "ltx_internal.hpp"
#include "ltx_loader.h"

namespace ltx {
std::string sha256_hex(const void* data, size_t n);
std::string normalize_name(const std::string& n);
void check_format_version(const json::Value& m);
}  // namespace ltx

static thread_local std::string g_loader_err;

struct BlobEntry {
    std::string name, norm, dtype, sha;
    uint64_t offset, nbytes;
};

struct ltx_blob {
    std::string manifest_text;
    std::vector<BlobEntry> entries;
    uint64_t total_bytes = 0, align = 64;
    int64_t block = -1;
    std::string blob_sha;
    void* data = nullptr;
    size_t size = 0;
};

enum class SlotState { Free, Filling, Ready, InUse };

struct HostSlot {
    void* mem = nullptr;
    SlotState state = SlotState::Free;
    size_t sched_pos = 0;
};

struct ltx_ring {
    HostSlot slots[2];
    uint64_t slot_bytes = 0;
    bool pinned = false;
    std::vector<ltx_blob*> blobs;
    std::vector<int> schedule;
    bool verify_first_touch = false;
    std::vector<char> verified;
    std::mutex mu;
    std::condition_variable cv;
    uint64_t reader_parks = 0, consumer_parks = 0, copy_ns = 0, verify_ns = 0;
    std::string reader_err;
    bool shutdown = false;
    uint32_t delay_us = 0;
    std::thread reader;
};

namespace {

[[noreturn]] void fail(const std::string& e) { throw ltx::Error(e); }

void set_state(HostSlot& s, SlotState to) {
    bool ok = (s.state == SlotState::Free && to == SlotState::Filling) ||
              (s.state == SlotState::Filling && to == SlotState::Ready) ||
              (s.state == SlotState::Ready && to == SlotState::InUse) ||
              (s.state == SlotState::InUse && to == SlotState::Free);
    if (!ok) {
        std::fprintf(stderr, "ltx ring: illegal slot transition %d -> %d\n", (int)s.state, (int)to);
        std::abort();
    }
    s.state = to;
}

uint64_t now_ns() {
    return (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

void reader_inner(ltx_ring* r) {
    for (size_t pos = 0; pos < r->schedule.size(); pos++) {
        HostSlot* slot = nullptr;
        {
            std::unique_lock<std::mutex> lk(r->mu);
            for (;;) {
                if (r->shutdown) fail("RingShutdown");
                for (auto& s : r->slots)
                    if (s.state == SlotState::Free) {
                        slot = &s;
                        break;
                    }
                if (slot) break;
                r->reader_parks++;
                r->cv.wait(lk);
            }
            set_state(*slot, SlotState::Filling);
            slot->sched_pos = pos;
        }
        if (r->delay_us) std::this_thread::sleep_for(std::chrono::microseconds(r->delay_us));
        ltx_blob* b = r->blobs[r->schedule[pos]];
        if (r->verify_first_touch && !r->verified[r->schedule[pos]]) {
            uint64_t t0 = now_ns();
            if (ltx::sha256_hex(b->data, b->size) != b->blob_sha) fail("BlobDigestMismatch");
            r->verified[r->schedule[pos]] = 1;
            r->verify_ns += now_ns() - t0;
        }
        uint64_t t0 = now_ns();
        std::memcpy(slot->mem, b->data, b->size);
        r->copy_ns += now_ns() - t0;
        {
            std::lock_guard<std::mutex> lk(r->mu);
            set_state(*slot, SlotState::Ready);
        }
        r->cv.notify_all();
    }
}

void reader_main(ltx_ring* r) {
    try {
        reader_inner(r);
    } catch (const std::exception& e) {
        {
            std::lock_guard<std::mutex> lk(r->mu);
            r->reader_err = e.what();
        }
        r->cv.notify_all();
    }
}

std::string read_file(const std::string& p) {
    std::ifstream f(p, std::ios::binary);
    if (!f) fail("cannot open " + p);
    std::stringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

}  // namespace

#define LOADER_GUARD(...)                      \
    try {                                       \
        __VA_ARGS__;                            \
        return 1;                               \
    } catch (const std::exception& ex) {        \
        g_loader_err = ex.what();               \
        return 0;                               \
    }

extern "C" {

const char* ltx_loader_last_error(void) { return g_loader_err.c_str(); }

int ltx_blob_open(const char* dir, ltx_blob** out) {
    ltx_blob* b = nullptr;
    try {
        if (!dir || !out) fail("NULL argument");
        *out = nullptr;
        b = new ltx_blob();
        std::string d(dir);
        b->manifest_text = read_file(d + "/blob_manifest.json");
        ltx::json::Value m = ltx::json::parse(b->manifest_text.c_str());
        try {
            ltx::check_format_version(m);
        } catch (const std::exception& ex) {
            fail(ex.what());
        }
        const int64_t total = m.at("total_bytes").as_int(), align = m.at("align").as_int();
        if (total < 0) fail("BlobSizeMismatch: negative total_bytes");
        if (align <= 0) fail("Misaligned: manifest align " + std::to_string(align));
        b->total_bytes = (uint64_t)total;
        b->align = (uint64_t)align;
        b->block = m.at("block").as_int();
        b->blob_sha = m.at("blob_sha256").as_str();
        for (const auto& e : m.at("entries").arr) {
            BlobEntry be;
            be.name = e.at("name").as_str();
            be.norm = ltx::normalize_name(be.name);
            be.dtype = e.at("dtype").as_str();
            const int64_t off = e.at("offset").as_int(), nb = e.at("nbytes").as_int();
            // entries lie inside the blob, with no sum that can wrap
            if (off < 0 || nb < 0 || (uint64_t)nb > b->total_bytes || (uint64_t)off > b->total_bytes - (uint64_t)nb)
                fail("TrailingBytes: entry beyond the blob: " + be.name);
            be.offset = (uint64_t)off;
            be.nbytes = (uint64_t)nb;
            if (const auto* s = e.get("sha256")) be.sha = s->as_str();
            b->entries.push_back(be);
        }
        std::string bp = d + "/blob.bin";
        struct stat st;
        if (::stat(bp.c_str(), &st) != 0) fail("cannot stat " + bp);
        if ((uint64_t)st.st_size != b->total_bytes) fail("BlobSizeMismatch");
        int fd = ::open(bp.c_str(), O_RDONLY);
        if (fd < 0) fail("cannot open " + bp);
        b->size = (size_t)st.st_size;
        if (b->size) {
            b->data = ::mmap(nullptr, b->size, PROT_READ, MAP_PRIVATE, fd, 0);
            if (b->data == MAP_FAILED) {
                b->data = nullptr;
                ::close(fd);
                fail("mmap failed for " + bp);
            }
        }
        ::close(fd);
        *out = b;
        return 1;
    } catch (const std::exception& ex) {
        g_loader_err = ex.what();
        delete b;
        return 0;
    }
}

void ltx_blob_close(ltx_blob* b) {
    if (!b) return;
    if (b->data) ::munmap(b->data, b->size);
    delete b;
}

int ltx_blob_check_layout(const ltx_blob* b) {
    LOADER_GUARD({
        if (!b) fail("NULL blob");
        uint64_t end = 0;
        for (const auto& e : b->entries) {
            if (e.offset % b->align != 0) fail("Misaligned: " + e.name);
            if (e.offset < end || e.offset - end >= b->align) fail("LayoutGap: " + e.name);
            end = e.offset + e.nbytes;
        }
        if (end != b->total_bytes) fail("TrailingBytes");
    })
}

int ltx_blob_verify(const ltx_blob* b) {
    LOADER_GUARD({
        if (!b) fail("NULL blob");
        if (ltx::sha256_hex(b->data, b->size) != b->blob_sha) fail("BlobDigestMismatch");
    })
}

const void* ltx_blob_data(const ltx_blob* b, uint64_t* bytes) {
    if (!b) return nullptr;
    if (bytes) *bytes = b->size;
    return b->data;
}

const char* ltx_blob_manifest_text(const ltx_blob* b) { return b ? b->manifest_text.c_str() : nullptr; }

int64_t ltx_blob_block_index(const ltx_blob* b) { return b ? b->block : -1; }

int ltx_blob_find(const ltx_blob* b, const char* want, uint64_t* offset, uint64_t* nbytes, char* dtype_out,
                  int dtype_cap) {
    LOADER_GUARD({
        if (!b || !want) fail("NULL argument");
        for (const auto& e : b->entries)
            if (e.norm == want) {
                if (offset) *offset = e.offset;
                if (nbytes) *nbytes = e.nbytes;
                if (dtype_out && dtype_cap > 0) std::snprintf(dtype_out, dtype_cap, "%s", e.dtype.c_str());
                return 1;
            }
        fail(std::string("MissingEntry: blob ") + std::to_string(b->block) + ": no entry named " + want);
    })
}

int ltx_ring_create(ltx_blob* const* blobs, int nblobs, const int* schedule, int nsched, int verify_first_touch,
                    uint64_t slot_bytes, int pinned, ltx_ring** out) {
    ltx_ring* r = nullptr;
    try {
        if (!blobs || nblobs <= 0 || !schedule || nsched < 0 || !out) fail("bad ring arguments");
        *out = nullptr;
        r = new ltx_ring();
        r->blobs.assign(blobs, blobs + nblobs);
        r->schedule.assign(schedule, schedule + nsched);
        r->verify_first_touch = verify_first_touch != 0;
        r->verified.assign(nblobs, 0);
        r->slot_bytes = slot_bytes;
        r->pinned = pinned != 0;
        for (auto& s : r->slots) {
            if (r->pinned) {
                HIPC(hipHostMalloc(&s.mem, slot_bytes ? slot_bytes : 1, hipHostMallocDefault));
            } else {
                s.mem = std::aligned_alloc(4096, ((slot_bytes ? slot_bytes : 1) + 4095) / 4096 * 4096);
                if (!s.mem) fail("slot allocation failed");
            }
        }
        *out = r;
        return 1;
    } catch (const std::exception& ex) {
        g_loader_err = ex.what();
        if (r) ltx_ring_destroy(r);
        return 0;
    }
}

int ltx_ring_static_check(const ltx_ring* r) {
    LOADER_GUARD({
        if (!r) fail("NULL ring");
        for (int bi : r->schedule) {
            if (bi < 0 || (size_t)bi >= r->blobs.size()) fail("ScheduleOutOfRange");
            if (r->blobs[bi]->total_bytes > r->slot_bytes) fail("SlotTooSmall");
        }
        // Serial consumer (one slot in use) + one reader (one slot filling):
        // peak occupancy min(2, schedule length) <= 2 slots.
    })
}

int ltx_ring_start(ltx_ring* r) {
    LOADER_GUARD({
        if (!r) fail("NULL ring");
        if (r->reader.joinable()) fail("reader already started");
        r->reader = std::thread(reader_main, r);
    })
}

int ltx_ring_acquire(ltx_ring* r, int pos, const void** mem, uint64_t* bytes) {
    LOADER_GUARD({
        if (!r) fail("NULL ring");
        std::unique_lock<std::mutex> lk(r->mu);
        for (;;) {
            if (!r->reader_err.empty()) fail(r->reader_err);
            for (auto& s : r->slots)
                if (s.state == SlotState::Ready && s.sched_pos == (size_t)pos) {
                    set_state(s, SlotState::InUse);
                    if (mem) *mem = s.mem;
                    if (bytes) *bytes = r->blobs[r->schedule[pos]]->size;
                    return 1;
                }
            if (r->shutdown) fail("RingShutdown");
            r->consumer_parks++;
            r->cv.wait(lk);
        }
    })
}

int ltx_ring_release(ltx_ring* r, int pos) {
    LOADER_GUARD({
        if (!r) fail("NULL ring");
        {
            std::lock_guard<std::mutex> lk(r->mu);
            HostSlot* hit = nullptr;
            for (auto& s : r->slots)
                if (s.state == SlotState::InUse && s.sched_pos == (size_t)pos) hit = &s;
            if (!hit) fail("release: schedule position is not in use");
            set_state(*hit, SlotState::Free);
        }
        r->cv.notify_all();
    })
}

void ltx_ring_abort(ltx_ring* r) {
    if (!r) return;
    {
        std::lock_guard<std::mutex> lk(r->mu);
        r->shutdown = true;
    }
    r->cv.notify_all();
}

int ltx_ring_stats(const ltx_ring* r, uint64_t* rp, uint64_t* cp, uint64_t* copy_ns, uint64_t* verify_ns) {
    LOADER_GUARD({
        if (!r) fail("NULL ring");
        if (rp) *rp = r->reader_parks;
        if (cp) *cp = r->consumer_parks;
        if (copy_ns) *copy_ns = r->copy_ns;
        if (verify_ns) *verify_ns = r->verify_ns;
    })
}

int ltx_ring_set_reader_delay_us(ltx_ring* r, uint32_t us) {
    LOADER_GUARD({
        if (!r) fail("NULL ring");
        r->delay_us = us;
    })
}

void ltx_ring_destroy(ltx_ring* r) {
    if (!r) return;
    ltx_ring_abort(r);
    if (r->reader.joinable()) r->reader.join();
    for (auto& s : r->slots) {
        if (!s.mem) continue;
        if (r->pinned)
            (void)hipHostFree(s.mem);
        else
            std::free(s.mem);
    }
    delete r;
}

}  // extern "C"
