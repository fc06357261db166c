// Engine object behind the C ABI: one HIP device, one stream, a registry of
// device buffers keyed by opaque int64 ids, a growable packing scratch and
// the pending batch of the record/commit API.
#pragma once

#include <memory>
#include <unordered_map>

#include "internal.h"

namespace rvc {

struct DevBuf {
  void* ptr = nullptr;
  size_t bytes = 0;
};

struct BatchOp {
  int op;
  long long a, b, c;
  long long p[20];  // p0..p10 of rvc_batch_add, or the longer parameter lists of the segment records
};

struct Engine {
  int device = 0;
  hipStream_t stream = nullptr;
  std::mutex mu;
  std::unordered_map<long long, DevBuf> bufs;
  long long next_id = 1;
  std::string device_name;
  // scratch for packed weights of op-level calls
  void* scratch = nullptr;
  size_t scratch_bytes = 0;
  // BiGRU exchange words + error flag of rvc_gru / rvc_batch_add_gru (kept
  // apart from the scratch, which later ops of a batch reuse), and whether a
  // launched GRU's flag still awaits its check after the next sync
  unsigned long long* gru_state = nullptr;
  bool gru_pending = false;
  // record/commit batch
  std::vector<BatchOp> batch;
  bool in_flight = false;
  // GPU-busy accounting behind rvc_ts_stats, on when RVC_TS=1 at creation:
  // every submission (a batch commit or a single-op call) is bracketed by
  // two events, resolved when the stats are read.
  bool ts_on = false;
  long long ts_busy_ns = 0, ts_submits = 0;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> ts_pending;

  Engine();
  ~Engine();

  long long add_buffer(void* p, size_t bytes);
  DevBuf& get(long long id);
  float* fptr(long long id, long long n_floats, const char* what);  // validates size
  void* scratch_for(size_t bytes);
  void sync();
  void ts_collect();  // sync, then fold the pending event pairs into ts_busy_ns
};

// Handle tables (handles are small sequential integers, never raw pointers,
// so a stale or forged handle is rejected instead of dereferenced).
Engine* engine_from_handle(long long h);

}  // namespace rvc
