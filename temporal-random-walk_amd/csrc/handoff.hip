// handoff.hip -- staged copies between caller host memory and HBM: walk
// buffers out to caller-owned host arrays, edge batches in.
//
// The reference fills its host walk set with one blocking cudaMemcpy per array
// into malloc'd memory (data/walk_set/walk_set_host.cu:55-85).  On this host a
// plain D2H copy into fresh pageable memory runs at a few GB/s: the runtime
// stages through its own small pinned buffer on one thread, and every 4 KiB
// page of the destination faults on first touch.  Here:
//  - destinations are 2 MiB-aligned and advised for transparent huge pages,
//    so first touch faults once per 2 MiB (they stay malloc-compatible:
//    free() releases them, as the C ABI promises);
//  - the copy is split into chunks that several host threads pull from one
//    queue; each thread owns a HIP stream and two pinned staging buffers, so
//    the DMA of its next chunk overlaps its memcpy of the current one, and
//    the page faults of the destination are taken by all threads at once.
// Host-pointer ingest (trw_add_edges) uses the same lanes in the other
// direction: the reference copies each batch array with one blocking
// cudaMemcpy (data/buffer.cuh:135-149).
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <memory>
#include <mutex>
#include <string>
#include <thread>

#include "engine.h"

namespace trw {

namespace {

constexpr size_t kHuge = size_t(2) << 20;
constexpr size_t kChunk = size_t(8) << 20;          // bytes per staged chunk
constexpr size_t kDirectBelow = size_t(32) << 20;   // smaller copies: one plain D2H
constexpr int kMaxThreads = 32;

int copy_threads() {
    static const int n = [] {
        int t = 8;
        if (const char* s = getenv("TRW_HOST_COPY_THREADS")) t = atoi(s);
        return std::max(1, std::min(t, kMaxThreads));
    }();
    return n;
}

}  // namespace

void* host_output_alloc(size_t bytes) {
    if (bytes < kHuge) {
        void* p = malloc(bytes ? bytes : 1);
        if (!p) throw std::bad_alloc();
        return p;
    }
    void* p = nullptr;
    if (posix_memalign(&p, kHuge, bytes) != 0 || !p) throw std::bad_alloc();
    // advisory only: without THP support the memory is simply 4 KiB-paged
    (void)madvise(p, (bytes + 4095) & ~size_t(4095), MADV_HUGEPAGE);
    return p;
}

HostLane::~HostLane() {
    if (stream) (void)hipStreamSynchronize(stream);
    for (auto& e : done)
        if (e) (void)hipEventDestroy(e);
    for (auto& b : stage)
        if (b) (void)hipHostFree(b);
    if (stream) (void)hipStreamDestroy(stream);
}

void HostLane::init() {
    if (stream) return;
    check_hip(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");
    for (auto& b : stage) check_hip(hipHostMalloc(&b, kChunk, hipHostMallocDefault), "hipHostMalloc");
    for (auto& e : done) check_hip(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate");
}

void Engine::copy_staged(const HostCopy* segs, size_t nseg, bool to_device) {
    copy_on_lanes(lanes, segs, nseg, to_device, true);
}

std::string Engine::join_prefetch() {
    if (!pf_pending) return "";
    if (pf_thread.joinable()) pf_thread.join();
    pf_pending = false;
    std::string err;
    err.swap(pf_error);
    return err;
}

void Engine::copy_on_lanes(std::vector<std::unique_ptr<HostLane>>& ls, const HostCopy* segs,
                           size_t nseg, bool to_device, bool engine_order) {
    size_t total = 0;
    for (size_t i = 0; i < nseg; ++i) total += segs[i].bytes;
    // earlier work on the engine stream may still read or write these buffers
    if (engine_order) sync();
    const auto t0 = std::chrono::steady_clock::now();
    const hipMemcpyKind kind = to_device ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost;

    if (total < kDirectBelow) {
        hipStream_t st = stream;
        if (!engine_order) {
            if (ls.empty()) ls.push_back(std::make_unique<HostLane>());
            ls[0]->init();
            st = ls[0]->stream;
        }
        for (size_t i = 0; i < nseg; ++i)
            if (segs[i].bytes)
                check_hip(hipMemcpyAsync(segs[i].dst, segs[i].src, segs[i].bytes, kind, st), "copy");
        check_hip(hipStreamSynchronize(st), "hipStreamSynchronize");
    } else {
        // chunk c of the whole transfer: segment seg_of[c], offset off_of[c]
        std::vector<size_t> seg_of, off_of;
        for (size_t i = 0; i < nseg; ++i)
            for (size_t o = 0; o < segs[i].bytes; o += kChunk) {
                seg_of.push_back(i);
                off_of.push_back(o);
            }
        const size_t nchunks = seg_of.size();
        const int nt = static_cast<int>(std::min<size_t>(copy_threads(), nchunks));
        while (ls.size() < static_cast<size_t>(nt)) ls.push_back(std::make_unique<HostLane>());
        for (int t = 0; t < nt; ++t) ls[t]->init();

        std::atomic<size_t> next{0};
        std::atomic<bool> failed{false};
        std::mutex err_mu;
        std::string err;
        auto chunk = [&](size_t c, size_t* n) {
            const HostCopy& s = segs[seg_of[c]];
            *n = std::min(kChunk, s.bytes - off_of[c]);
            return s;
        };
        // device -> host: the DMA of a lane's next chunk into one staging
        // buffer overlaps its memcpy of the other out to the destination
        auto to_host = [&](HostLane& ln) {
            size_t held[2];
            size_t bytes_of[2] = {0, 0};
            auto issue = [&](int b) -> bool {
                const size_t c = next.fetch_add(1);
                if (c >= nchunks || failed.load()) return false;
                size_t n;
                const HostCopy& s = chunk(c, &n);
                check_hip(hipMemcpyAsync(ln.stage[b], static_cast<const char*>(s.src) + off_of[c], n,
                                         hipMemcpyDeviceToHost, ln.stream),
                          "D2H stage");
                check_hip(hipEventRecord(ln.done[b], ln.stream), "hipEventRecord");
                held[b] = c;
                bytes_of[b] = n;
                return true;
            };
            bool more[2] = {issue(0), false};
            if (more[0]) more[1] = issue(1);
            int live = more[0] + more[1];
            for (int b = 0; live > 0; b ^= 1) {
                if (!more[b]) continue;
                check_hip(hipEventSynchronize(ln.done[b]), "hipEventSynchronize");
                const size_t c = held[b];
                memcpy(static_cast<char*>(segs[seg_of[c]].dst) + off_of[c], ln.stage[b], bytes_of[b]);
                more[b] = issue(b);
                if (!more[b]) --live;
            }
        };
        // host -> device: a lane fills one staging buffer while the DMA of
        // the other is in flight, waiting only before it refills a buffer
        auto to_dev = [&](HostLane& ln) {
            bool pending[2] = {false, false};
            for (int b = 0;; b ^= 1) {
                const size_t c = next.fetch_add(1);
                if (c >= nchunks || failed.load()) break;
                size_t n;
                const HostCopy& s = chunk(c, &n);
                if (pending[b]) check_hip(hipEventSynchronize(ln.done[b]), "hipEventSynchronize");
                memcpy(ln.stage[b], static_cast<const char*>(s.src) + off_of[c], n);
                check_hip(hipMemcpyAsync(static_cast<char*>(s.dst) + off_of[c], ln.stage[b], n,
                                         hipMemcpyHostToDevice, ln.stream),
                          "H2D stage");
                check_hip(hipEventRecord(ln.done[b], ln.stream), "hipEventRecord");
                pending[b] = true;
            }
            check_hip(hipStreamSynchronize(ln.stream), "hipStreamSynchronize");
        };
        auto worker = [&](int t) {
            HostLane& ln = *ls[t];
            try {
                check_hip(hipSetDevice(device), "hipSetDevice");
                if (to_device) to_dev(ln);
                else to_host(ln);
            } catch (const std::exception& ex) {
                failed.store(true);
                (void)hipStreamSynchronize(ln.stream);  // no DMA may outlive the call
                std::lock_guard<std::mutex> g(err_mu);
                if (err.empty()) err = ex.what();
            }
        };
        std::vector<std::thread> pool;
        pool.reserve(nt - 1);
        for (int t = 1; t < nt; ++t) pool.emplace_back(worker, t);
        worker(0);
        for (auto& th : pool) th.join();
        if (failed.load()) throw std::runtime_error("host copy: " + err);
    }
    const double ms =
        std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    if (!to_device && engine_order) {
        timings.handoff_ms = ms;
        timings.handoff_bytes = total;
    }
}

}  // namespace trw
