/*
 * vx_stream_policy.h -- what a wait or a free does on the caller's stream.
 *
 * A host program may hand the library a HIP stream for the calling thread
 * (vx_cuda_set_stream / vx_hip_set_stream). Launches then go on that stream,
 * and a wait covers that stream only. While that stream is being captured
 * into a hipGraph, nothing that blocks the host can run: a wait, a copy
 * between host and HBM, or a free that must wait first. The library then
 * stops with a message naming the capture instead of failing inside HIP.
 * Memory the library allocated in stream order (hipMallocAsync on the
 * caller's stream) is freed in stream order on that stream, with no wait,
 * which a capture can hold.
 *
 * The same decisions as reference runtime/vx_stream_policy.h:23-58 (the
 * outcomes are observable through the ABI, so they must agree); kept free
 * of HIP so tests/native/stream_policy_test.cpp checks them on any machine.
 */
#ifndef VX_AMD_STREAM_POLICY_H
#define VX_AMD_STREAM_POLICY_H

namespace vx {

enum class WaitAction {
  kDevice, /* no caller stream: wait for every kernel of the device */
  kStream, /* wait for the caller's stream only */
  kRefuse, /* the caller's stream is capturing: a wait cannot be recorded */
};

inline WaitAction wait_action(bool has_stream, bool capturing) {
  if (!has_stream) {
    return WaitAction::kDevice;
  }
  return capturing ? WaitAction::kRefuse : WaitAction::kStream;
}

enum class FreeAction {
  kAfterDeviceWait, /* wait for the device, then hipFree */
  kAfterStreamWait, /* wait for the caller's stream, then hipFree */
  kOnStream,        /* hipFreeAsync on the stream the memory came from */
  kRefuse,          /* capturing, and the memory needs a wait first */
};

/* `stream_ordered`: the memory came from hipMallocAsync on a caller's stream;
 * it is freed in that stream's order whatever stream is set now. */
inline FreeAction free_action(bool has_stream, bool capturing,
                              bool stream_ordered) {
  if (stream_ordered) {
    return FreeAction::kOnStream;
  }
  if (!has_stream) {
    return FreeAction::kAfterDeviceWait;
  }
  return capturing ? FreeAction::kRefuse : FreeAction::kAfterStreamWait;
}

} // namespace vx

#endif /* VX_AMD_STREAM_POLICY_H */
