// Host -> device transfer engine for expert pages (host code; part of the C ABI).
//
// Pinned host memory comes from hipHostMalloc. The engine owns one worker thread and a
// priority queue of chunk copies: a task (dst, src, bytes) is split into num_chunks chunks of
// whole elements; the worker takes the highest-priority chunk, copies it with
// hipMemcpyAsync on the task's stream and waits for that copy (an event on the stream), so a
// more urgent task submitted meanwhile runs before the remaining chunks of a long one. The
// first chunk of a task stamps its start time and the last its end time; waiters block on a
// condition variable until the last chunk lands.
//
// Reference: HtoDTransferEngine, specmoe/backend/htod_transfer_engine.py:73-520 (priority
// order :29-63, chunking :313-369, worker :405-489, completion and timing :371-403,491-520),
// and pin_memory_allocator.py:7-28 (libcudart cudaMallocHost) for the pinned allocation.
#include "../../include/specmoe_mi355x.h"
#include "smx_kernels.h"

#include <chrono>
#include <condition_variable>
#include <cstring>
#include <map>
#include <mutex>
#include <queue>
#include <string>
#include <thread>
#include <vector>

namespace {

using Clock = std::chrono::steady_clock;

// Priority classes, most urgent first (reference TASK_PRIORITY_MAPPING).
int priority_of(int type) {
  switch (type) {
    case SMX_H2D_HIDDEN: return 1;
    case SMX_H2D_KV_CACHE: return 2;
    case SMX_H2D_DRAFT_KV_CACHE: return 3;
    default: return 4;  // SMX_H2D_WEIGHT
  }
}

struct Chunk {
  int priority;
  int64_t layer;   // 0 sorts after every other layer (reference TransferTask.__lt__)
  int64_t index;   // 1-based chunk index within its task
  int64_t total;
  int64_t seq;     // submission order, the last tie-break
  char* dst;
  const char* src;
  size_t bytes;
  hipStream_t stream;
  std::string task;
  int64_t generation;  // the task submission this chunk belongs to
};

// Strict weak order for the queue: true when a runs after b.
struct RunsAfter {
  bool operator()(const Chunk& a, const Chunk& b) const {
    if (a.priority != b.priority) return a.priority > b.priority;
    if (a.layer != b.layer) {
      if (a.layer == 0) return true;
      if (b.layer == 0) return false;
      return a.layer > b.layer;
    }
    if (a.index != b.index) return a.index > b.index;
    return a.seq > b.seq;
  }
};

struct TaskState {
  int64_t generation = 0;
  bool done = false;
  int status = SMX_OK;
  bool weight = false;
  Clock::time_point start{}, end{};
};

}  // namespace

struct smx_h2d_engine {
  std::mutex mu;
  std::condition_variable cv_work;  // worker: queue non-empty, enabled, or stopping
  std::condition_variable cv_done;  // waiters: a task completed
  std::priority_queue<Chunk, std::vector<Chunk>, RunsAfter> queue;
  std::map<std::string, TaskState> tasks;
  bool running = true;
  bool enabled = true;
  int64_t seq = 0;
  int64_t generations = 0;
  int device = 0;
  hipEvent_t done_event = nullptr;
  std::thread worker;

  void run() {
    (void)hipSetDevice(device);
    for (;;) {
      Chunk c;
      {
        std::unique_lock<std::mutex> lk(mu);
        cv_work.wait(lk, [&] { return !running || (enabled && !queue.empty()); });
        if (!running) return;
        c = queue.top();
        queue.pop();
        if (c.index == 1) {
          auto it = tasks.find(c.task);
          if (it != tasks.end() && it->second.generation == c.generation) it->second.start = Clock::now();
        }
      }
      int status = static_cast<int>(hipMemcpyAsync(c.dst, c.src, c.bytes, hipMemcpyHostToDevice, c.stream));
      if (status == hipSuccess) status = static_cast<int>(hipEventRecord(done_event, c.stream));
      if (status == hipSuccess) status = static_cast<int>(hipEventSynchronize(done_event));
      std::lock_guard<std::mutex> lk(mu);
      auto it = tasks.find(c.task);
      if (it == tasks.end() || it->second.generation != c.generation) continue;  // cleared or resubmitted
      TaskState& t = it->second;
      if (status != hipSuccess && t.status == SMX_OK) t.status = status;
      if (c.index == c.total) {
        t.end = Clock::now();
        t.done = true;
        cv_done.notify_all();
      }
    }
  }
};

extern "C" {

int smx_host_alloc(size_t bytes, void** ptr) {
  if (!ptr || bytes == 0) return SMX_ERR_INVALID_ARG;
  *ptr = nullptr;
  return static_cast<int>(hipHostMalloc(ptr, bytes, hipHostMallocPortable));
}

int smx_host_free(void* ptr) {
  if (!ptr) return SMX_OK;
  return static_cast<int>(hipHostFree(ptr));
}

int smx_h2d_engine_create(smx_h2d_engine** out) {
  if (!out) return SMX_ERR_INVALID_ARG;
  *out = nullptr;
  auto* e = new smx_h2d_engine();
  int rc = static_cast<int>(hipGetDevice(&e->device));
  if (rc == hipSuccess) rc = static_cast<int>(hipEventCreateWithFlags(&e->done_event, hipEventDisableTiming));
  if (rc != hipSuccess) {
    delete e;
    return rc;
  }
  e->worker = std::thread([e] { e->run(); });
  *out = e;
  return SMX_OK;
}

int smx_h2d_engine_destroy(smx_h2d_engine* e) {
  if (!e) return SMX_OK;
  {
    std::lock_guard<std::mutex> lk(e->mu);
    e->running = false;
    e->cv_work.notify_all();
  }
  e->worker.join();
  (void)hipEventDestroy(e->done_event);
  delete e;
  return SMX_OK;
}

int smx_h2d_submit(smx_h2d_engine* e, int task_type, const char* task_id, void* dst,
                   const void* src, size_t bytes, size_t elem_bytes, int64_t num_chunks,
                   int64_t layer_id, void* stream) {
  if (!e || !task_id || !dst || !src || bytes == 0 || elem_bytes == 0 || bytes % elem_bytes != 0 ||
      num_chunks < 1 || task_type < SMX_H2D_HIDDEN || task_type > SMX_H2D_WEIGHT)
    return SMX_ERR_INVALID_ARG;
  const int64_t elems = static_cast<int64_t>(bytes / elem_bytes);
  if (num_chunks > elems) return SMX_ERR_INVALID_ARG;
  std::lock_guard<std::mutex> lk(e->mu);
  TaskState& t = e->tasks[task_id];
  t = TaskState{};
  t.generation = ++e->generations;
  t.weight = task_type == SMX_H2D_WEIGHT;
  // whole elements per chunk; the first `rem` chunks take one more (reference :342-350)
  const int64_t base = elems / num_chunks, rem = elems % num_chunks;
  int64_t pos = 0;
  for (int64_t i = 0; i < num_chunks; ++i) {
    const int64_t n = base + (i < rem ? 1 : 0);
    Chunk c;
    c.priority = priority_of(task_type);
    c.layer = layer_id;
    c.index = i + 1;
    c.total = num_chunks;
    c.seq = e->seq++;
    c.dst = static_cast<char*>(dst) + pos * static_cast<int64_t>(elem_bytes);
    c.src = static_cast<const char*>(src) + pos * static_cast<int64_t>(elem_bytes);
    c.bytes = static_cast<size_t>(n) * elem_bytes;
    c.stream = static_cast<hipStream_t>(stream);
    c.task = task_id;
    c.generation = t.generation;
    e->queue.push(c);
    pos += n;
  }
  e->cv_work.notify_one();
  return SMX_OK;
}

int smx_h2d_wait(smx_h2d_engine* e, const char* task_id, double timeout_s, double* seconds) {
  if (!e || !task_id) return SMX_ERR_INVALID_ARG;
  std::unique_lock<std::mutex> lk(e->mu);
  auto it = e->tasks.find(task_id);
  if (it == e->tasks.end()) return SMX_ERR_NOT_FOUND;
  const std::string key = task_id;
  auto ready = [&] {
    auto f = e->tasks.find(key);
    return f == e->tasks.end() || f->second.done;
  };
  if (timeout_s < 0) {
    e->cv_done.wait(lk, ready);
  } else if (!e->cv_done.wait_for(lk, std::chrono::duration<double>(timeout_s), ready)) {
    return SMX_ERR_TIMEOUT;
  }
  it = e->tasks.find(key);
  if (it == e->tasks.end()) return SMX_ERR_NOT_FOUND;  // cleared while waiting
  if (seconds) {
    *seconds = it->second.weight ? std::chrono::duration<double>(it->second.end - it->second.start).count()
                                 : -1.0;
  }
  return it->second.status;
}

int smx_h2d_has_task(smx_h2d_engine* e, const char* task_id) {
  if (!e || !task_id) return 0;
  std::lock_guard<std::mutex> lk(e->mu);
  return e->tasks.count(task_id) ? 1 : 0;
}

int smx_h2d_clear(smx_h2d_engine* e, const char* task_id) {
  if (!e || !task_id) return SMX_ERR_INVALID_ARG;
  std::lock_guard<std::mutex> lk(e->mu);
  e->tasks.erase(task_id);
  e->cv_done.notify_all();
  return SMX_OK;
}

int smx_h2d_set_enabled(smx_h2d_engine* e, int enabled) {
  if (!e) return SMX_ERR_INVALID_ARG;
  std::lock_guard<std::mutex> lk(e->mu);
  e->enabled = enabled != 0;
  e->cv_work.notify_all();
  return SMX_OK;
}

int smx_h2d_pending(smx_h2d_engine* e) {
  if (!e) return 0;
  std::lock_guard<std::mutex> lk(e->mu);
  return static_cast<int>(e->queue.size());
}

}  // extern "C"
