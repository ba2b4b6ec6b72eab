// tierlift.hip -- TierLift: the bounded host reducer of the edge-record stream.
//
// Reference role: SpillEdgeSink feeding ExternalHashPruneReducer
// (shear-core/src/algorithm/pipnn/spill_hashprune.rs: shard routing
// flush_pending_edges :569-614, shard buffers and segment flush :616-658 and
// :727-757, part files :772-830, manifest :832-851, shard-by-shard reduction
// :853-892).
//
//   push     the caller's stream records an event; a side stream (default
//            priority) waits on it, sorts the batch by (src, dst) on the
//            device and drops exact repeats of a record (the same pair seen
//            forward and reverse in one batch: a reservoir ignores a repeat),
//            so leaf compute goes on while a slot drains;
//   worker   a host thread takes the slots in order, copies each batch's
//            records into its pinned staging slot and appends each shard's run
//            (the batch is in source order, src / shard_points) to that
//            shard's blocks of 1,000,000 records, shards in parallel;
//   spill    past 7/8 of the host budget the worker hands the shard with the
//            most buffered records to a spill thread and goes on routing (it
//            waits only past the budget itself): each of the shard's blocks
//            becomes one segment, sorted by src (counting sort, stable), placed
//            in the shard's part files (rolled over past 4 GiB) at offsets
//            fixed before the parallel writes;
//   finish   the manifest is written, then shard by shard the spilled
//            segments (read straight into the pinned slots) and the buffered
//            blocks go back to the device on the copy stream into two device
//            buffers in turn, while the caller's stream rebases sources to the
//            shard and merges the other buffer with the HashPrune reservoir
//            kernels; each shard's reservoirs are exported into the caller's
//            neighbour table.
//
// A reservoir's final state depends only on its record set (HashPrune with
// backfill and evidence policies off), so the table equals one in-HBM
// reduction of the same records, whatever was spilled.
#include <fcntl.h>
#include <sys/mman.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <condition_variable>
#include <deque>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include <hipcub/hipcub.hpp>

#include "hashprune_kernels.h"
#include "tessa_device.h"

namespace tessa {
tessa_status hashprune_insert_async(tessa_hashprune *hp, const tessa_edge_record *records, uint64_t count,
                                    hipStream_t hs);
}

namespace {

struct Rec {
    uint32_t src, dst;
    uint16_t hash, flags;
    float dist;
};
static_assert(sizeof(Rec) == 16, "SpillRecord16");

constexpr uint64_t kBlockRecords = 1000000;                   // segment cap, spill_hashprune.rs:25,:500-505
constexpr uint64_t kBlockBytes = kBlockRecords * sizeof(Rec);
constexpr uint64_t kHugePage = 2ull << 20;
constexpr uint64_t kBlockAlloc = (kBlockBytes + kHugePage - 1) / kHugePage * kHugePage;
constexpr uint64_t kPartMaxBytes = 4ull * 1024 * 1024 * 1024;  // DEFAULT_PART_MAX_BYTES :27
constexpr uint64_t kUploadRecords = 1ull << 26;               // records per reservoir merge at finish (1 GiB)
constexpr uint64_t kCountingSortMaxShard = 1ull << 24;        // larger shards sort by comparison
constexpr uint64_t kEagerSpillBlocks = 16;                    // an early-spilled shard's job size (256 MB)

struct Shard {
    std::vector<Rec *> blocks;  // kBlockRecords each; the last one partly filled
    uint64_t n = 0;             // buffered records
    uint32_t part = 0;          // current part file index
    uint64_t part_bytes = 0;    // bytes in the current part file
    int fd = -1;
};

struct Segment {
    uint32_t shard, file;
    uint64_t offset, bytes, records;
    uint32_t src_min, src_max;
};

// Per-slot device workspace of the batch sort (base 256-byte aligned).
struct SlotWs {
    uint64_t *keys_in, *keys_out, *vals_in, *vals_out;
    uint4 *recs, *out;
    uint8_t *flag;
    unsigned long long *count;  // [0] kept records, [1] first bad record (index << 32 | src)
    void *temp;
};
uint64_t ws_align(uint64_t x) { return (x + 255) & ~(uint64_t)255; }
SlotWs slot_ws(void *base, uint64_t n) {
    char *p = static_cast<char *>(base);
    SlotWs w{};
    uint64_t at = 0;
    auto take = [&](uint64_t bytes) {
        void *q = p + at;
        at += ws_align(bytes);
        return q;
    };
    w.keys_in = static_cast<uint64_t *>(take(n * 8));
    w.keys_out = static_cast<uint64_t *>(take(n * 8));
    w.vals_in = static_cast<uint64_t *>(take(n * 8));
    w.vals_out = static_cast<uint64_t *>(take(n * 8));
    w.recs = static_cast<uint4 *>(take(n * 16));
    w.out = static_cast<uint4 *>(take(n * 16));
    w.flag = static_cast<uint8_t *>(take(n));
    w.count = static_cast<unsigned long long *>(take(16));
    w.temp = p + at;
    return w;
}
uint64_t slot_ws_fixed_bytes(uint64_t n) {
    return 4 * ws_align(n * 8) + 2 * ws_align(n * 16) + ws_align(n) + ws_align(16);
}
size_t sort_temp_bytes(uint64_t n) {
    size_t a = 0, b = 0;
    (void)hipcub::DeviceRadixSort::SortPairs(nullptr, a, (const uint64_t *)nullptr, (uint64_t *)nullptr,
                                             (const uint64_t *)nullptr, (uint64_t *)nullptr, (int)n, 0, 64);
    (void)hipcub::DeviceSelect::Flagged(nullptr, b, (const uint4 *)nullptr, (const uint8_t *)nullptr, (uint4 *)nullptr,
                                        (unsigned long long *)nullptr, (int)n);
    return a > b ? a : b;
}
int key_bits_for(uint64_t num_points) {
    int b = 1;
    while (b < 32 && (1ull << b) < num_points) ++b;
    return 32 + b;
}

// A shard's buffered records handed to the spill thread.
struct SpillJob {
    uint32_t shard;
    std::vector<Rec *> blocks;
    uint64_t n;
};

// A batch as sort keys (src, dst) and values (hash, flags, dist).
// A batch as sort keys (src, dst) and values (hash, flags, dist); *bad gets
// the first record with src >= num_points as (index << 32 | src).
__global__ void tl_keys_kernel(const uint4 *rec, uint64_t n, uint32_t num_points, uint64_t *keys, uint64_t *vals,
                               unsigned long long *bad) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint4 r = rec[i];
    keys[i] = ((uint64_t)r.x << 32) | r.y;
    vals[i] = ((uint64_t)r.w << 32) | r.z;
    if (r.x >= num_points) atomicMin(bad, (unsigned long long)((i << 32) | r.x));
}

__global__ void tl_init_kernel(unsigned long long *bad) { *bad = ~0ull; }

// The sorted batch back as records; flag[i] marks a record that differs from
// its predecessor (the first of a run of repeats).
__global__ void tl_unkey_kernel(const uint64_t *keys, const uint64_t *vals, uint64_t n, uint4 *rec, uint8_t *flag) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t k = keys[i], v = vals[i];
    rec[i] = make_uint4((uint32_t)(k >> 32), (uint32_t)k, (uint32_t)v, (uint32_t)(v >> 32));
    flag[i] = i == 0 || keys[i - 1] != k || vals[i - 1] != v;
}

__global__ void rebase_src_kernel(uint4 *rec, uint64_t n, uint32_t lo) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) rec[i].x -= lo;
}

tessa_status tl_status(int32_t code, const char *fmt, ...) {
    tessa_status s{};
    s.code = code;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(s.msg, sizeof(s.msg), fmt, ap);
    va_end(ap);
    return s;
}

double now_s() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

template <typename F>
void parallel_for(uint32_t T, F &&f) {
    if (T <= 1) {
        f(0u);
        return;
    }
    std::vector<std::thread> pool;
    pool.reserve(T - 1);
    for (uint32_t w = 1; w < T; ++w) pool.emplace_back(f, w);
    f(0u);
    for (auto &th : pool) th.join();
}

}  // namespace

struct tessa_tierlift {
    tessa_tierlift_config cfg{};
    int device = 0;
    uint32_t shards = 0;
    uint32_t threads = 1;
    std::string dir, stem;  // part files: dir/stem_shardSSSSS_partPPP.log
    // D2H staging: per slot the device sort buffers (keys and values in and
    // out, the records in order, repeat flags, the kept records, their count,
    // the sort / select temporary), the pinned host slot and its count
    hipStream_t copy_stream = nullptr, d2h_stream = nullptr;
    Rec *pinned[2] = {nullptr, nullptr};
    uint64_t *pinned_count = nullptr;  // [2]
    void *dev_ws[2] = {nullptr, nullptr};
    size_t sort_temp_bytes = 0;
    hipEvent_t ready[2] = {nullptr, nullptr}, counted[2] = {nullptr, nullptr}, copied[2] = {nullptr, nullptr};
    uint64_t slot_n[2] = {0, 0}, slot_seq[2] = {0, 0};
    bool slot_full[2] = {false, false};
    int next_slot = 0;
    uint64_t next_seq = 0, copied_seq = 0;
    // host worker and spill thread (mu guards the slots, the block pool, the
    // spill queue, segments and error)
    std::mutex mu;
    std::condition_variable cv;
    std::thread worker, spiller;
    bool stopping = false, finished = false;
    std::string error;
    std::deque<SpillJob> jobs;
    bool spilling = false;  // the spill thread holds a job
    uint32_t keep_shards = 0;  // shards [keep_shards, shards) are spilled from the start
    // shard blocks (routing: worker), part files (spill thread, then finish)
    std::vector<Shard> shard;
    std::vector<Rec *> free_blocks;
    uint64_t blocks_in_use = 0, blocks_allocated = 0;
    std::vector<Segment> segments;
    tessa_tierlift_stats stats{};
};

namespace {

std::string part_path(const tessa_tierlift *t, uint32_t shard, uint32_t part) {
    char tail[64];
    snprintf(tail, sizeof(tail), "_shard%05u_part%03u.log", shard, part);
    return t->dir + "/" + t->stem + tail;
}

// Block pool; the caller holds t->mu.
Rec *take_block(tessa_tierlift *t) {
    Rec *b = nullptr;
    if (!t->free_blocks.empty()) {
        b = t->free_blocks.back();
        t->free_blocks.pop_back();
    } else {
        // 2 MB aligned with huge pages: routing writes each new block once,
        // and 4 KB first-touch faults would dominate that copy
        void *q = nullptr;
        if (posix_memalign(&q, kHugePage, kBlockAlloc) != 0 || !q) return nullptr;
        (void)madvise(q, kBlockAlloc, MADV_HUGEPAGE);
        b = static_cast<Rec *>(q);
        t->blocks_allocated += 1;
        t->stats.host_peak_bytes = std::max(t->stats.host_peak_bytes, t->blocks_allocated * kBlockBytes);
    }
    t->blocks_in_use += 1;
    return b;
}

void give_block(tessa_tierlift *t, Rec *b) {
    t->free_blocks.push_back(b);
    t->blocks_in_use -= 1;
}

// Writes a job's records (a shard's detached blocks) as segments, one per
// block, sorted by src, to the shard's part files, then returns the blocks to
// the pool.  Spill thread only (and the part-file state is the spill
// thread's until finish).
bool spill_job(tessa_tierlift *t, SpillJob &job, std::string &err) {
    const uint32_t s = job.shard;
    Shard &sh = t->shard[s];
    const double t0 = now_s();
    const uint32_t nb = (uint32_t)job.blocks.size();
    struct Place {
        uint32_t file;
        int fd;
        uint64_t offset, records;
    };
    std::vector<Place> place(nb);
    std::vector<int> to_close;  // part files rolled over here: closed after the writes
    for (uint32_t b = 0; b < nb; ++b) {
        const uint64_t n = std::min<uint64_t>(kBlockRecords, job.n - (uint64_t)b * kBlockRecords);
        const uint64_t bytes = n * sizeof(Rec);
        if (sh.fd < 0 || sh.part_bytes + bytes > kPartMaxBytes) {
            if (sh.fd >= 0) {
                to_close.push_back(sh.fd);
                sh.fd = -1;
                sh.part += 1;
            }
            const std::string path = part_path(t, s, sh.part);
            sh.fd = open(path.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
            sh.part_bytes = 0;
            if (sh.fd < 0) {
                for (int fd : to_close) close(fd);
                err = "TierLift spill: cannot create " + path;
                return false;
            }
        }
        place[b] = Place{sh.part, sh.fd, sh.part_bytes, n};
        sh.part_bytes += bytes;
    }
    const uint64_t lo = (uint64_t)s * t->cfg.shard_points;
    const uint64_t span = std::min<uint64_t>(t->cfg.shard_points, t->cfg.num_points - lo);
    std::vector<uint32_t> smin(nb), smax(nb);
    const uint32_t T = std::max(1u, std::min<uint32_t>(t->threads, nb));
    std::vector<char> failed(T, 0);
    parallel_for(T, [&](uint32_t w) {
        std::vector<Rec> out(kBlockRecords);
        std::vector<uint32_t> hist(span <= kCountingSortMaxShard ? span + 1 : 0);
        for (uint32_t b = w; b < nb; b += T) {
            const Rec *in = job.blocks[b];
            const uint64_t n = place[b].records;
            if (!hist.empty()) {
                std::fill(hist.begin(), hist.end(), 0u);
                for (uint64_t i = 0; i < n; ++i) hist[in[i].src - lo + 1] += 1;
                for (uint64_t k = 1; k <= span; ++k) hist[k] += hist[k - 1];
                for (uint64_t i = 0; i < n; ++i) out[hist[in[i].src - lo]++] = in[i];
            } else {
                std::copy(in, in + n, out.begin());
                std::stable_sort(out.begin(), out.begin() + n, [](const Rec &a, const Rec &c) { return a.src < c.src; });
            }
            smin[b] = n ? out[0].src : 0u;
            smax[b] = n ? out[n - 1].src : 0u;
            const char *p = reinterpret_cast<const char *>(out.data());
            uint64_t left = n * sizeof(Rec), off = place[b].offset;
            while (left) {
                const ssize_t wr = pwrite(place[b].fd, p, left, (off_t)off);
                if (wr <= 0) {
                    failed[w] = 1;
                    break;
                }
                p += wr;
                off += (uint64_t)wr;
                left -= (uint64_t)wr;
            }
        }
    });
    for (int fd : to_close) close(fd);
    for (char f : failed)
        if (f) {
            err = "TierLift spill: short write to a part file of shard " + std::to_string(s);
            return false;
        }
    std::lock_guard<std::mutex> lk(t->mu);
    for (uint32_t b = 0; b < nb; ++b) {
        const uint64_t bytes = place[b].records * sizeof(Rec);
        t->segments.push_back(Segment{s, place[b].file, place[b].offset, bytes, place[b].records, smin[b], smax[b]});
        t->stats.spilled_records += place[b].records;
        t->stats.spilled_bytes += bytes;
        t->stats.segments += 1;
        give_block(t, job.blocks[b]);
    }
    job.blocks.clear();
    t->stats.spill_s += now_s() - t0;
    return true;
}

void spiller_main(tessa_tierlift *t) {
    for (;;) {
        SpillJob job;
        {
            std::unique_lock<std::mutex> lk(t->mu);
            t->cv.wait(lk, [&] { return !t->jobs.empty() || t->stopping; });
            if (t->jobs.empty()) return;
            job = std::move(t->jobs.front());
            t->jobs.pop_front();
            t->spilling = true;
        }
        std::string err;
        const bool ok = spill_job(t, job, err);
        {
            std::lock_guard<std::mutex> lk(t->mu);
            if (!ok) {
                if (t->error.empty()) t->error = err;
                for (Rec *b : job.blocks) give_block(t, b);  // not written: back to the pool
            }
            t->spilling = false;
        }
        t->cv.notify_all();
    }
}

// Appends a batch in source order to its shards: each shard's run (found by
// binary search) goes after what the shard holds, shards over the threads.
bool route_sorted(tessa_tierlift *t, const Rec *r, uint64_t n, std::string &err) {
    const double t0 = now_s();
    const uint32_t S = t->shards;
    const uint64_t sp = t->cfg.shard_points;
    std::vector<uint64_t> first(S + 1), at(S);
    for (uint32_t s = 0; s < S; ++s) {
        const uint64_t lo = (uint64_t)s * sp;
        first[s] = (uint64_t)(std::lower_bound(r, r + n, lo, [](const Rec &a, uint64_t v) { return a.src < v; }) - r);
    }
    first[S] = n;
    for (uint32_t s = 0; s < S; ++s) {
        Shard &sh = t->shard[s];
        at[s] = sh.n;
        const uint64_t need = sh.n + (first[s + 1] - first[s]);
        while (sh.blocks.size() * kBlockRecords < need) {
            Rec *b;
            {
                std::lock_guard<std::mutex> lk(t->mu);
                b = take_block(t);
            }
            if (!b) {
                err = "TierLift: host block allocation failed";
                return false;
            }
            sh.blocks.push_back(b);
        }
        sh.n = need;
    }
    const uint32_t T = n < (1u << 16) ? 1u : std::min<uint32_t>(t->threads, S);
    parallel_for(T, [&](uint32_t w) {
        for (uint32_t s = w; s < S; s += T) {
            Shard &sh = t->shard[s];
            uint64_t pos = at[s];
            for (uint64_t i = first[s]; i < first[s + 1];) {
                const uint64_t off = pos % kBlockRecords;
                const uint64_t m = std::min<uint64_t>(kBlockRecords - off, first[s + 1] - i);
                std::memcpy(sh.blocks[pos / kBlockRecords] + off, r + i, m * sizeof(Rec));
                pos += m;
                i += m;
            }
        }
    });
    t->stats.route_s += now_s() - t0;
    return true;
}

// After a batch is routed: a shard past the ones the expected stream leaves
// room for goes to the spill thread once it has kEagerSpillBlocks blocks;
// past 7/8 of the budget the biggest shard does (one job at a time) and
// routing goes on; past the budget itself the worker waits for the spill to
// return blocks.
bool keep_budget(tessa_tierlift *t, std::string &err) {
    const uint64_t hard = t->cfg.host_budget_bytes, soft = hard - hard / 8;
    std::unique_lock<std::mutex> lk(t->mu);
    if (t->cfg.expected_records && t->stats.records) {
        // the expected stream as the batches so far thin it (repeats dropped)
        const double kept = (double)t->stats.unique_records / (double)t->stats.records;
        const double bytes = (double)t->cfg.expected_records * kept * (double)sizeof(Rec);
        t->keep_shards =
            bytes > (double)soft ? (uint32_t)((double)t->shards * (double)soft / bytes) : t->shards;
    }
    if (!t->dir.empty() && t->keep_shards < t->shards && t->jobs.empty() && !t->spilling) {
        uint32_t big = t->keep_shards;
        for (uint32_t s = big + 1; s < t->shards; ++s)
            if (t->shard[s].n > t->shard[big].n) big = s;
        Shard &sh = t->shard[big];
        if (sh.n >= kEagerSpillBlocks * kBlockRecords) {
            t->jobs.push_back(SpillJob{big, std::move(sh.blocks), sh.n});
            sh.blocks.clear();
            sh.n = 0;
            t->cv.notify_all();
        }
    }
    for (;;) {
        const uint64_t used = t->blocks_in_use * kBlockBytes;
        if (!t->error.empty()) {
            err = t->error;
            return false;
        }
        if (used <= soft) return true;
        if (t->dir.empty()) {
            if (used <= hard) return true;
            char m[240];
            snprintf(m, sizeof(m),
                     "TierLift host budget of %llu bytes exceeded and no spill path given "
                     "overflow_flags=0x%llx overflow_labels=WORKSPACE_BUDGET",
                     (unsigned long long)hard, (unsigned long long)TESSA_OVF_WORKSPACE_BUDGET);
            err = m;
            return false;
        }
        if (t->jobs.empty() && !t->spilling) {
            uint32_t big = 0;
            for (uint32_t s = 1; s < t->shards; ++s)
                if (t->shard[s].n > t->shard[big].n) big = s;
            Shard &sh = t->shard[big];
            if (sh.n == 0) return true;  // everything buffered is being written
            t->jobs.push_back(SpillJob{big, std::move(sh.blocks), sh.n});
            sh.blocks.clear();
            sh.n = 0;
            t->cv.notify_all();
        }
        if (used <= hard) return true;
        t->cv.wait(lk);
    }
}

// The D2H copy of slot `slot`'s kept records, once its sort is done (waits
// for it); false (with t->error set) on a failed sort or D2H, or an
// out-of-range record.  Worker only.
bool start_copy(tessa_tierlift *t, int slot, uint64_t &m) {
    bool ok = hipEventSynchronize(t->counted[slot]) == hipSuccess;
    m = t->pinned_count[2 * slot];
    const uint64_t bad = t->pinned_count[2 * slot + 1];
    {
        std::lock_guard<std::mutex> lk(t->mu);
        t->copied_seq = t->slot_seq[slot];  // the caller's records are read
        if (!ok && t->error.empty()) t->error = "TierLift: sorting a record batch failed";
        if (ok && bad != ~0ull && t->error.empty()) {
            char msg[200];
            snprintf(msg, sizeof(msg), "Spill reducer encountered edge p=%u outside shard range [0, %llu)",
                     (uint32_t)bad, (unsigned long long)t->cfg.num_points);
            t->error = msg;
        }
        ok = t->error.empty();
    }
    t->cv.notify_all();
    if (!ok) return false;
    const SlotWs w = slot_ws(t->dev_ws[slot], t->cfg.staging_records);
    if (hipMemcpyAsync(t->pinned[slot], w.out, m * sizeof(Rec), hipMemcpyDeviceToHost, t->d2h_stream) != hipSuccess ||
        hipEventRecord(t->copied[slot], t->d2h_stream) != hipSuccess) {
        std::lock_guard<std::mutex> lk(t->mu);
        if (t->error.empty()) t->error = "TierLift: D2H copy of a record batch failed";
        return false;
    }
    return true;
}

void worker_main(tessa_tierlift *t) {
    (void)hipSetDevice(t->device);
    int slot = 0;
    bool started[2] = {false, false};
    uint64_t kept[2] = {0, 0};
    for (;;) {
        {
            std::unique_lock<std::mutex> lk(t->mu);
            t->cv.wait(lk, [&] { return t->slot_full[slot] || t->stopping; });
            if (!t->slot_full[slot]) return;
        }
        bool ok = started[slot] || start_copy(t, slot, kept[slot]);
        started[slot] = false;
        // the other slot's copy goes while this one is routed, if it is
        // filled and sorted already
        const int other = slot ^ 1;
        bool other_full;
        {
            std::lock_guard<std::mutex> lk(t->mu);
            other_full = t->slot_full[other];
        }
        if (ok && other_full && hipEventQuery(t->counted[other]) == hipSuccess)
            started[other] = start_copy(t, other, kept[other]);
        if (ok) {
            std::string err;
            ok = hipEventSynchronize(t->copied[slot]) == hipSuccess;
            if (!ok) err = "TierLift: D2H copy of a record batch failed";
            if (ok) {
                t->stats.records += t->slot_n[slot];
                t->stats.unique_records += kept[slot];
                ok = route_sorted(t, t->pinned[slot], kept[slot], err);
            }
            if (ok) ok = keep_budget(t, err);
            if (!ok) {
                std::lock_guard<std::mutex> lk(t->mu);
                if (t->error.empty()) t->error = err;
            }
        }
        {
            std::lock_guard<std::mutex> lk(t->mu);
            t->slot_full[slot] = false;
        }
        t->cv.notify_all();
        slot ^= 1;
    }
}

}  // namespace

extern "C" {

tessa_status tessa_tierlift_create(const tessa_tierlift_config *cfg, tessa_tierlift **out) {
    if (!cfg || !out) return tl_status(TESSA_ERR_INVALID_ARGUMENT, "tierlift: null argument");
    *out = nullptr;
    if (cfg->num_points == 0 || cfg->num_points > 0xffffffffull || cfg->shard_points == 0 || cfg->l_max == 0 ||
        cfg->staging_records == 0)
        return tl_status(TESSA_ERR_INVALID_ARGUMENT,
                         "tierlift: num_points in [1, 2^32), shard_points, l_max and staging_records must be > 0");
    if (cfg->l_max > tessa::kHpMaxLMax)
        return tl_status(TESSA_ERR_UNSUPPORTED, "tierlift: l_max=%u above %u", cfg->l_max, tessa::kHpMaxLMax);
    auto *t = new (std::nothrow) tessa_tierlift();
    if (!t) return tl_status(TESSA_ERR_OUT_OF_MEMORY, "tierlift: host allocation failed");
    t->cfg = *cfg;
    t->cfg.spill_base = nullptr;  // copied below; the caller's string need not outlive the call
    t->shards = (uint32_t)((cfg->num_points + cfg->shard_points - 1) / cfg->shard_points);
    t->threads = cfg->threads ? cfg->threads : std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (cfg->spill_base && cfg->spill_base[0]) {
        // part files sit next to the base path, named after its stem (spill_hashprune.rs:823-830)
        const std::string base = cfg->spill_base;
        const size_t slash = base.find_last_of('/');
        t->dir = slash == std::string::npos ? std::string(".") : slash == 0 ? std::string("/") : base.substr(0, slash);
        std::string name = slash == std::string::npos ? base : base.substr(slash + 1);
        const size_t dot = name.find_last_of('.');
        if (dot != std::string::npos && dot > 0) name = name.substr(0, dot);
        t->stem = name.empty() ? std::string("candidate") : name;
    }
    t->shard.resize(t->shards);
    // the shards a stream of expected_records leaves room for (7/8 of the budget)
    t->keep_shards = t->shards;
    const uint64_t expect_bytes = cfg->expected_records * sizeof(Rec);
    const uint64_t soft = cfg->host_budget_bytes - cfg->host_budget_bytes / 8;
    if (expect_bytes > soft)
        t->keep_shards = (uint32_t)((double)t->shards * (double)soft / (double)expect_bytes);
    if (cfg->staging_records >= (1ull << 31)) {
        delete t;
        return tl_status(TESSA_ERR_UNSUPPORTED, "tierlift: staging_records %llu (limit 2^31-1)",
                         (unsigned long long)cfg->staging_records);
    }
    t->sort_temp_bytes = sort_temp_bytes(cfg->staging_records);
    const uint64_t ws_bytes = slot_ws_fixed_bytes(cfg->staging_records) + t->sort_temp_bytes;
    bool ok = hipGetDevice(&t->device) == hipSuccess &&
              hipStreamCreateWithFlags(&t->copy_stream, hipStreamNonBlocking) == hipSuccess &&
              hipStreamCreateWithFlags(&t->d2h_stream, hipStreamNonBlocking) == hipSuccess &&
              hipHostMalloc((void **)&t->pinned_count, 4 * sizeof(uint64_t)) == hipSuccess;
    for (int i = 0; ok && i < 2; ++i)
        ok = hipHostMalloc((void **)&t->pinned[i], cfg->staging_records * sizeof(Rec)) == hipSuccess &&
             hipMalloc(&t->dev_ws[i], ws_bytes) == hipSuccess &&
             hipEventCreateWithFlags(&t->ready[i], hipEventDisableTiming) == hipSuccess &&
             hipEventCreateWithFlags(&t->counted[i], hipEventDisableTiming) == hipSuccess &&
             hipEventCreateWithFlags(&t->copied[i], hipEventDisableTiming) == hipSuccess;
    if (!ok) {
        tessa_tierlift_destroy(t);
        return tl_status(TESSA_ERR_OUT_OF_MEMORY,
                         "tierlift: staging set-up (pinned 2 x %llu records, device 2 x %llu bytes) failed",
                         (unsigned long long)cfg->staging_records, (unsigned long long)ws_bytes);
    }
    t->stats.shards = t->shards;
    t->stats.threads = t->threads;
    t->worker = std::thread(worker_main, t);
    t->spiller = std::thread(spiller_main, t);
    *out = t;
    return tessa_status{};
}

tessa_status tessa_tierlift_push(tessa_tierlift *t, const tessa_edge_record *records, uint64_t count, void *stream,
                                 uint64_t *seq_out) {
    if (!t) return tl_status(TESSA_ERR_INVALID_ARGUMENT, "tierlift is null");
    if (count && !records) return tl_status(TESSA_ERR_INVALID_ARGUMENT, "tierlift: null records");
    if (t->finished) return tl_status(TESSA_ERR_INVALID_ARGUMENT, "tierlift: push after finish");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    uint64_t done = 0;
    while (done < count) {
        const uint64_t n = std::min<uint64_t>(t->cfg.staging_records, count - done);
        const int slot = t->next_slot;
        {
            std::unique_lock<std::mutex> lk(t->mu);
            t->cv.wait(lk, [&] { return !t->slot_full[slot] || !t->error.empty(); });
            if (!t->error.empty()) return tl_status(TESSA_ERR_INVALID_ARGUMENT, "%s", t->error.c_str());
        }
        // the side stream waits for the caller's stream (never the other
        // way round), sorts the batch by (src, dst), drops repeats and
        // copies the count of kept records (and the first out-of-range
        // record) to the host
        const SlotWs w = slot_ws(t->dev_ws[slot], t->cfg.staging_records);
        hipStream_t cs = t->copy_stream;
        const uint32_t grid = (uint32_t)((n + 255) / 256);
        size_t tb = t->sort_temp_bytes;
        bool ok = hipEventRecord(t->ready[slot], s) == hipSuccess &&
                  hipStreamWaitEvent(cs, t->ready[slot], 0) == hipSuccess;
        if (ok) {
            hipLaunchKernelGGL(tl_init_kernel, dim3(1), dim3(1), 0, cs, w.count + 1);
            hipLaunchKernelGGL(tl_keys_kernel, dim3(grid), dim3(256), 0, cs,
                               reinterpret_cast<const uint4 *>(records + done), n, (uint32_t)t->cfg.num_points,
                               w.keys_in, w.vals_in, w.count + 1);
            ok = hipGetLastError() == hipSuccess &&
                 hipcub::DeviceRadixSort::SortPairs(w.temp, tb, w.keys_in, w.keys_out, w.vals_in, w.vals_out, (int)n,
                                                    0, key_bits_for(t->cfg.num_points), cs) == hipSuccess;
        }
        if (ok) {
            hipLaunchKernelGGL(tl_unkey_kernel, dim3(grid), dim3(256), 0, cs, w.keys_out, w.vals_out, n, w.recs,
                               w.flag);
            tb = t->sort_temp_bytes;
            ok = hipGetLastError() == hipSuccess &&
                 hipcub::DeviceSelect::Flagged(w.temp, tb, w.recs, w.flag, w.out, w.count, (int)n, cs) == hipSuccess &&
                 hipMemcpyAsync(t->pinned_count + 2 * slot, w.count, 16, hipMemcpyDeviceToHost, cs) == hipSuccess &&
                 hipEventRecord(t->counted[slot], cs) == hipSuccess;
        }
        if (!ok) return tl_status(TESSA_ERR_HIP, "tierlift: enqueueing the batch sort and D2H failed");
        {
            std::lock_guard<std::mutex> lk(t->mu);
            t->slot_n[slot] = n;
            t->slot_seq[slot] = ++t->next_seq;
            t->slot_full[slot] = true;
        }
        t->cv.notify_all();
        t->next_slot ^= 1;
        done += n;
        t->stats.pushes += 1;
    }
    if (seq_out) *seq_out = t->next_seq;
    return tessa_status{};
}

tessa_status tessa_tierlift_copied(tessa_tierlift *t, uint64_t *seq) {
    if (!t || !seq) return tl_status(TESSA_ERR_INVALID_ARGUMENT, "tierlift: null argument");
    std::lock_guard<std::mutex> lk(t->mu);
    *seq = t->copied_seq;
    if (!t->error.empty()) return tl_status(TESSA_ERR_INVALID_ARGUMENT, "%s", t->error.c_str());
    return tessa_status{};
}

tessa_status tessa_tierlift_wait(tessa_tierlift *t, uint64_t seq) {
    if (!t) return tl_status(TESSA_ERR_INVALID_ARGUMENT, "tierlift is null");
    std::unique_lock<std::mutex> lk(t->mu);
    t->cv.wait(lk, [&] { return t->copied_seq >= seq || !t->error.empty(); });
    if (!t->error.empty()) return tl_status(TESSA_ERR_INVALID_ARGUMENT, "%s", t->error.c_str());
    return tessa_status{};
}

tessa_status tessa_tierlift_finish(tessa_tierlift *t, uint32_t *targets, uint32_t *counts, void *stream,
                                   tessa_tierlift_stats *stats_out) {
    if (!t || !targets || !counts) return tl_status(TESSA_ERR_INVALID_ARGUMENT, "tierlift: null argument");
    if (t->finished) return tl_status(TESSA_ERR_INVALID_ARGUMENT, "tierlift: finish called twice");
    {
        std::unique_lock<std::mutex> lk(t->mu);
        t->cv.wait(lk, [&] { return (!t->slot_full[0] && !t->slot_full[1] && t->jobs.empty() && !t->spilling) ||
                                    !t->error.empty(); });
        if (!t->error.empty()) return tl_status(TESSA_ERR_INVALID_ARGUMENT, "%s", t->error.c_str());
    }
    t->finished = true;  // the worker is idle from here on; no push is accepted
    const double t0 = now_s();
    for (Shard &sh : t->shard)
        if (sh.fd >= 0) {
            close(sh.fd);
            sh.fd = -1;
        }
    if (!t->dir.empty() && !t->segments.empty()) {
        std::sort(t->segments.begin(), t->segments.end(), [](const Segment &a, const Segment &b) {
            return a.shard != b.shard ? a.shard < b.shard : a.file != b.file ? a.file < b.file : a.offset < b.offset;
        });
        const std::string mpath = t->dir + "/candidate_segments.manifest";
        FILE *m = fopen(mpath.c_str(), "w");
        if (!m) return tl_status(TESSA_ERR_INVALID_ARGUMENT, "TierLift spill: cannot write %s", mpath.c_str());
        for (const Segment &g : t->segments)
            fprintf(m, "%u,%u,%llu,%llu,%llu,%u,%u,1\n", g.shard, g.file, (unsigned long long)g.offset,
                    (unsigned long long)g.bytes, (unsigned long long)g.records, g.src_min, g.src_max);
        if (fclose(m) != 0)
            return tl_status(TESSA_ERR_INVALID_ARGUMENT, "TierLift spill: writing %s failed", mpath.c_str());
    }
    hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
    hipStream_t cs = t->copy_stream;  // idle now: the H2D side of the pipeline
    const uint32_t sp = (uint32_t)std::min<uint64_t>(t->cfg.shard_points, t->cfg.num_points);
    tessa_hashprune *hp = nullptr;
    tessa_status st = tessa_hashprune_create(sp, t->cfg.l_max, &hp);
    if (st.code) return st;
    // two device buffers: the copy stream fills one while the caller's stream
    // merges the other; up[b] marks buffer b filled, merged[b] merged
    uint4 *dev[2] = {nullptr, nullptr};
    hipEvent_t up[2] = {nullptr, nullptr}, merged[2] = {nullptr, nullptr};
    uint32_t *t_tmp = nullptr, *c_tmp = nullptr;
    const uint64_t dev_cap = std::max<uint64_t>(kUploadRecords, t->cfg.staging_records);
    bool ok = hipMalloc(&dev[0], dev_cap * sizeof(Rec)) == hipSuccess &&
              hipMalloc(&dev[1], dev_cap * sizeof(Rec)) == hipSuccess &&
              hipMalloc(&t_tmp, (uint64_t)sp * t->cfg.l_max * 4) == hipSuccess &&
              hipMalloc(&c_tmp, (uint64_t)sp * 4) == hipSuccess;
    for (int i = 0; ok && i < 2; ++i)
        ok = hipEventCreateWithFlags(&up[i], hipEventDisableTiming) == hipSuccess &&
             hipEventCreateWithFlags(&merged[i], hipEventDisableTiming) == hipSuccess &&
             hipEventRecord(merged[i], hs) == hipSuccess && hipEventRecord(t->copied[i], cs) == hipSuccess;
    if (!ok)
        st = tl_status(TESSA_ERR_OUT_OF_MEMORY, "tierlift: reduction buffers (2 x %llu records) failed",
                       (unsigned long long)dev_cap);
    int slot = 0, cur = 0;
    uint64_t fill = 0;
    size_t seg = 0;
    // buffer cur may be filled once its previous merge is done
    if (!st.code && hipStreamWaitEvent(cs, merged[cur], 0) != hipSuccess)
        st = tl_status(TESSA_ERR_HIP, "tierlift: stream wait failed");
    for (uint32_t s = 0; s < t->shards && !st.code; ++s) {
        const uint32_t lo = (uint32_t)((uint64_t)s * t->cfg.shard_points);
        const uint32_t n_s = (uint32_t)std::min<uint64_t>(t->cfg.shard_points, t->cfg.num_points - lo);
        // the filled part of buffer cur to the reservoirs (records routed to
        // this shard are in range: no read-back of the range check)
        auto merge = [&]() -> tessa_status {
            if (!fill) return tessa_status{};
            if (hipEventRecord(up[cur], cs) != hipSuccess || hipStreamWaitEvent(hs, up[cur], 0) != hipSuccess)
                return tl_status(TESSA_ERR_HIP, "tierlift: event failed");
            hipLaunchKernelGGL(rebase_src_kernel, dim3((uint32_t)((fill + 255) / 256)), dim3(256), 0, hs, dev[cur],
                               fill, lo);
            tessa_status s2 = tessa::hashprune_insert_async(hp, reinterpret_cast<const tessa_edge_record *>(dev[cur]),
                                                            fill, hs);
            if (s2.code) return s2;
            if (hipEventRecord(merged[cur], hs) != hipSuccess) return tl_status(TESSA_ERR_HIP, "tierlift: event failed");
            cur ^= 1;
            fill = 0;
            if (hipStreamWaitEvent(cs, merged[cur], 0) != hipSuccess)
                return tl_status(TESSA_ERR_HIP, "tierlift: stream wait failed");
            return tessa_status{};
        };
        // m records into pinned slot `slot` by fill_slot(dst), then H2D into buffer cur
        auto add = [&](uint64_t n, auto &&fill_slot) -> tessa_status {
            for (uint64_t a = 0; a < n;) {
                const uint64_t m = std::min<uint64_t>({t->cfg.staging_records, dev_cap - fill, n - a});
                if (hipEventSynchronize(t->copied[slot]) != hipSuccess)
                    return tl_status(TESSA_ERR_HIP, "tierlift: H2D of shard %u records failed", s);
                if (!fill_slot(t->pinned[slot], a, m))
                    return tl_status(TESSA_ERR_INVALID_ARGUMENT, "TierLift spill: short read of a segment of shard %u", s);
                if (hipMemcpyAsync(dev[cur] + fill, t->pinned[slot], m * sizeof(Rec), hipMemcpyHostToDevice, cs) !=
                        hipSuccess ||
                    hipEventRecord(t->copied[slot], cs) != hipSuccess)
                    return tl_status(TESSA_ERR_HIP, "tierlift: H2D of shard %u records failed", s);
                slot ^= 1;
                fill += m;
                a += m;
                if (fill == dev_cap) {
                    tessa_status s2 = merge();
                    if (s2.code) return s2;
                }
            }
            return tessa_status{};
        };
        st = tessa_hashprune_clear(hp, stream);
        // spilled segments of this shard (manifest order), read into the
        // pinned slots, then its buffered blocks
        for (; !st.code && seg < t->segments.size() && t->segments[seg].shard == s; ++seg) {
            const Segment &g = t->segments[seg];
            const std::string path = part_path(t, g.shard, g.file);
            const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
            if (fd < 0) {
                st = tl_status(TESSA_ERR_INVALID_ARGUMENT, "TierLift spill: cannot reopen %s", path.c_str());
                break;
            }
            st = add(g.records, [&](Rec *dst, uint64_t a, uint64_t m) {
                const uint32_t T = m < (1u << 16) ? 1u : t->threads;
                std::vector<char> bad(T, 0);
                parallel_for(T, [&](uint32_t w) {
                    const uint64_t x = m * w / T, y = m * (w + 1) / T;
                    char *p = reinterpret_cast<char *>(dst + x);
                    uint64_t left = (y - x) * sizeof(Rec), off = g.offset + (a + x) * sizeof(Rec);
                    while (left) {
                        const ssize_t r = pread(fd, p, left, (off_t)off);
                        if (r <= 0) {
                            bad[w] = 1;
                            return;
                        }
                        p += r;
                        off += (uint64_t)r;
                        left -= (uint64_t)r;
                    }
                });
                for (char b : bad)
                    if (b) return false;
                return true;
            });
            close(fd);
            t->stats.reread_records += g.records;
        }
        Shard &sh = t->shard[s];
        for (size_t b = 0; b < sh.blocks.size() && !st.code; ++b) {
            const Rec *src = sh.blocks[b];
            st = add(std::min<uint64_t>(kBlockRecords, sh.n - b * kBlockRecords), [&](Rec *dst, uint64_t a, uint64_t m) {
                const uint32_t T = m < (1u << 18) ? 1u : t->threads;
                parallel_for(T, [&](uint32_t w) {
                    const uint64_t x = m * w / T, y = m * (w + 1) / T;
                    std::memcpy(dst + x, src + a + x, (y - x) * sizeof(Rec));
                });
                return true;
            });
        }
        if (!st.code) st = merge();
        if (!st.code) st = tessa_hashprune_neighbors(hp, t_tmp, nullptr, nullptr, c_tmp, stream);
        if (!st.code &&
            (hipMemcpyAsync(targets + (uint64_t)lo * t->cfg.l_max, t_tmp, (uint64_t)n_s * t->cfg.l_max * 4,
                            hipMemcpyDeviceToDevice, hs) != hipSuccess ||
             hipMemcpyAsync(counts + lo, c_tmp, (uint64_t)n_s * 4, hipMemcpyDeviceToDevice, hs) != hipSuccess))
            st = tl_status(TESSA_ERR_HIP, "tierlift: shard export copy failed");
        // the blocks were copied into the pinned slots on the host: free now
        {
            std::lock_guard<std::mutex> lk(t->mu);
            for (Rec *b : sh.blocks) give_block(t, b);
        }
        sh.blocks.clear();
        sh.n = 0;
    }
    if (!st.code && hipStreamSynchronize(hs) != hipSuccess) st = tl_status(TESSA_ERR_HIP, "tierlift: sync failed");
    (void)hipStreamSynchronize(hs);
    (void)hipStreamSynchronize(cs);
    for (int i = 0; i < 2; ++i) {
        if (dev[i]) (void)hipFree(dev[i]);
        if (up[i]) (void)hipEventDestroy(up[i]);
        if (merged[i]) (void)hipEventDestroy(merged[i]);
    }
    if (t_tmp) (void)hipFree(t_tmp);
    if (c_tmp) (void)hipFree(c_tmp);
    tessa_hashprune_destroy(hp);
    for (Rec *b : t->free_blocks) std::free(b);
    t->free_blocks.clear();
    t->blocks_allocated = 0;
    t->stats.reduce_s = now_s() - t0;
    if (stats_out) *stats_out = t->stats;
    return st;
}

tessa_status tessa_tierlift_destroy(tessa_tierlift *t) {
    if (!t) return tessa_status{};
    {
        std::lock_guard<std::mutex> lk(t->mu);
        t->stopping = true;
    }
    t->cv.notify_all();
    if (t->worker.joinable()) t->worker.join();
    if (t->spiller.joinable()) t->spiller.join();
    for (Shard &sh : t->shard) {
        if (sh.fd >= 0) close(sh.fd);
        for (Rec *b : sh.blocks) std::free(b);
    }
    for (Rec *b : t->free_blocks) std::free(b);
    if (t->copy_stream) (void)hipStreamSynchronize(t->copy_stream);
    if (t->d2h_stream) (void)hipStreamSynchronize(t->d2h_stream);
    for (int i = 0; i < 2; ++i) {
        if (t->pinned[i]) (void)hipHostFree(t->pinned[i]);
        if (t->dev_ws[i]) (void)hipFree(t->dev_ws[i]);
        if (t->ready[i]) (void)hipEventDestroy(t->ready[i]);
        if (t->counted[i]) (void)hipEventDestroy(t->counted[i]);
        if (t->copied[i]) (void)hipEventDestroy(t->copied[i]);
    }
    if (t->pinned_count) (void)hipHostFree(t->pinned_count);
    if (t->copy_stream) (void)hipStreamDestroy(t->copy_stream);
    if (t->d2h_stream) (void)hipStreamDestroy(t->d2h_stream);
    delete t;
    return tessa_status{};
}

}  // extern "C"
