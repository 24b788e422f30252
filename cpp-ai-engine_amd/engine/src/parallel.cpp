// parallel.cpp -- a small persistent host thread pool behind engine::parallel
// (the reference's include/engine/parallel.hpp API). Workers sleep on a
// condition variable; a call publishes one job (the body and its chunk
// bounds), the caller runs chunk 0 and the workers the rest, and the caller
// waits for the chunk counter. Calls are serialised by a mutex; a nested call
// runs inline.
#include "engine/parallel.hpp"

#include <algorithm>
#include <condition_variable>
#include <cstdlib>
#include <exception>
#include <mutex>
#include <thread>
#include <vector>

namespace engine {
namespace parallel {

namespace {

thread_local bool t_inside = false;

struct Pool {
    std::mutex call;  // one parallel_for at a time
    std::mutex m;
    std::condition_variable wake, done;
    std::vector<std::thread> workers;
    size_t threads = 1;
    // the current job
    const std::function<void(size_t, size_t)>* body = nullptr;
    std::vector<size_t> bounds;  // chunk c is [bounds[c], bounds[c + 1])
    size_t next = 0, finished = 0, chunks = 0;
    uint64_t generation = 0;
    std::exception_ptr error;
    bool stop = false;

    Pool() {
        size_t n = std::max<size_t>(1, std::thread::hardware_concurrency());
        if (const char* env = std::getenv("ENGINE_NUM_THREADS")) {
            const long v = std::atol(env);
            if (v > 0) n = size_t(v);
        }
        resize(n);
    }
    ~Pool() { resize(0); }

    void run_chunk(size_t c) {
        t_inside = true;
        try {
            (*body)(bounds[c], bounds[c + 1]);
        } catch (...) {
            std::lock_guard<std::mutex> lk(m);
            if (!error) error = std::current_exception();
        }
        t_inside = false;
    }

    void worker() {
        uint64_t seen = 0;
        std::unique_lock<std::mutex> lk(m);
        for (;;) {
            wake.wait(lk, [&] { return stop || (generation != seen && next < chunks); });
            if (stop) return;
            while (next < chunks) {
                const size_t c = next++;
                lk.unlock();
                run_chunk(c);
                lk.lock();
                if (++finished == chunks) done.notify_all();
            }
            seen = generation;
        }
    }

    // 0 joins every worker (destruction); otherwise n - 1 workers.
    void resize(size_t n) {
        {
            std::lock_guard<std::mutex> lk(m);
            stop = true;
        }
        wake.notify_all();
        for (std::thread& t : workers) t.join();
        workers.clear();
        stop = false;
        threads = std::max<size_t>(n, 1);
        if (n == 0) return;
        for (size_t i = 1; i < threads; ++i) workers.emplace_back([this] { worker(); });
    }
};

Pool& pool() {
    static Pool p;
    return p;
}

}  // namespace

size_t num_threads() { return pool().threads; }

void set_num_threads(size_t threads) {
    Pool& p = pool();
    std::lock_guard<std::mutex> call(p.call);
    p.resize(std::max<size_t>(threads, 1));
}

bool inside_parallel_region() { return t_inside; }

void parallel_for(size_t count, size_t min_per_thread,
                  const std::function<void(size_t begin, size_t end)>& body) {
    if (count == 0) return;
    Pool& p = pool();
    const size_t per = std::max<size_t>(min_per_thread, 1);
    size_t chunks = std::min(p.threads, (count + per - 1) / per);
    if (chunks <= 1 || t_inside) {
        const bool outer = !t_inside;
        t_inside = true;
        try {
            body(0, count);
        } catch (...) {
            if (outer) t_inside = false;
            throw;
        }
        if (outer) t_inside = false;
        return;
    }
    std::lock_guard<std::mutex> call(p.call);
    chunks = std::min(chunks, p.threads);
    {
        std::lock_guard<std::mutex> lk(p.m);
        p.body = &body;
        p.bounds.resize(chunks + 1);
        for (size_t c = 0; c <= chunks; ++c) p.bounds[c] = count * c / chunks;
        p.chunks = chunks;
        p.next = 1;  // chunk 0 is the caller's
        p.finished = 0;
        p.error = nullptr;
        ++p.generation;
    }
    p.wake.notify_all();
    p.run_chunk(0);
    std::unique_lock<std::mutex> lk(p.m);
    while (p.next < p.chunks) {  // help with chunks no worker has taken yet
        const size_t c = p.next++;
        lk.unlock();
        p.run_chunk(c);
        lk.lock();
        ++p.finished;
    }
    ++p.finished;  // chunk 0
    p.done.wait(lk, [&] { return p.finished == p.chunks; });
    p.body = nullptr;
    p.chunks = 0;
    if (p.error) {
        std::exception_ptr e = p.error;
        p.error = nullptr;
        std::rethrow_exception(e);
    }
}

}  // namespace parallel
}  // namespace engine
