// fmxq_device_state.hip -- device memory the library keeps for the life of the
// process in file-scope __device__ variables rather than hipMalloc:
//   - the index-error flags that gather kernels raise and fmxq_device_error
//     reads and clears: kFlagSlots words per device.  Word 0 is the graph word:
//     launches enqueued while their stream is being captured into a graph get
//     it, because the graph may be replayed on any stream.  Words 1 ..
//     kFlagSlots - 1 belong to streams, in order of first use (past that many
//     streams on one device, slots are shared in turn);
//   - `scratch`, the fixed workspace of fmxq_switch_glu_noalloc
//     (FMXQ_NOALLOC_SCRATCH_BYTES), for callers that cannot allocate.
// Each GPU holds its own copy of both at its own address.  In host code the
// variables' names are host-side stand-ins, not device addresses, so each is
// resolved once per device with hipGetSymbolAddress (with that device current)
// and only the resolved pointers are ever handed to kernels or copies.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>

#include "../../include/fmxq.h"
#include "fmxq_host.hpp"

// 16 KiB per device: enough streams that a process sharing a word between two
// of them is not a practical case.
constexpr int kFlagSlots = 4096;
static __device__ __align__(256) uint32_t index_flag[kFlagSlots];
static __device__ __align__(256) unsigned char scratch[FMXQ_NOALLOC_SCRATCH_BYTES];

namespace {

struct DeviceState {
  uint32_t* flag = nullptr;  // kFlagSlots words
  void* scratch = nullptr;
  std::map<hipStream_t, int> slot;
  int next_slot = 0;
};
// One entry per device, created on the device's first use.  Map nodes keep
// their addresses when other devices are added, so a DeviceState pointer stays
// valid without the lock held.
std::mutex g_state_mu;
std::map<int, DeviceState> g_state;

// The current device's resolved addresses, looked up on its first use.
int current_state(DeviceState** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fmxq::fail(FMXQ_ERR_DEVICE, "hipGetDevice failed");
  std::lock_guard<std::mutex> lk(g_state_mu);
  DeviceState& st = g_state[dev];
  if (!st.flag) {
    void* f = nullptr;
    void* s = nullptr;
    if (int rc = fmxq::hip_status(hipGetSymbolAddress(&f, HIP_SYMBOL(index_flag)),
                                  "hipGetSymbolAddress(index flag)"))
      return rc;
    if (int rc = fmxq::hip_status(hipGetSymbolAddress(&s, HIP_SYMBOL(scratch)),
                                  "hipGetSymbolAddress(scratch)"))
      return rc;
    st.scratch = s;
    st.flag = static_cast<uint32_t*>(f);  // set last: a non-null flag means resolved
  }
  *out = &st;
  return FMXQ_OK;
}

// The stream's own word (1 .. kFlagSlots - 1), assigned on first use.
uint32_t* stream_word(DeviceState* st, hipStream_t stream) {
  std::lock_guard<std::mutex> lk(g_state_mu);
  auto it = st->slot.find(stream);
  if (it == st->slot.end())
    it = st->slot.emplace(stream, 1 + st->next_slot++ % (kFlagSlots - 1)).first;
  return st->flag + it->second;
}

}  // namespace

namespace fmxq {

int device_flag(hipStream_t stream, uint32_t** out) {
  DeviceState* st = nullptr;
  if (int rc = current_state(&st)) return rc;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone) {
    *out = st->flag;  // the graph word
    return FMXQ_OK;
  }
  *out = stream_word(st, stream);
  return FMXQ_OK;
}

int device_flags_to_check(hipStream_t stream, uint32_t** own, uint32_t** graph) {
  DeviceState* st = nullptr;
  if (int rc = current_state(&st)) return rc;
  *own = stream_word(st, stream);
  *graph = st->flag;
  return FMXQ_OK;
}

int noalloc_scratch(void** out) {
  DeviceState* st = nullptr;
  if (int rc = current_state(&st)) return rc;
  *out = st->scratch;
  return FMXQ_OK;
}

}  // namespace fmxq
