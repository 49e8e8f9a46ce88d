// workspace.hpp - device scratch memory for the work one C-ABI call enqueues on a stream (internal to libnnh).
//
// Each (device, stream) pair has one scratch buffer. By default the library owns it: allocated on first use,
// grown on demand and kept until the process ends. A caller may instead register a buffer of its own for the
// stream (nnh_set_workspace); from then on calls on that stream take their scratch from it and never allocate,
// and a call that needs more than it holds fails before launching anything.
//   * A call takes the buffer with a StreamWorkspace for as long as it enqueues work; work on one stream runs in
//     order, so the next call on that stream may reuse the buffer at once. No call frees memory on its way
//     (hipFreeAsync makes the host wait until the stream reaches it, which would keep the host from running
//     ahead of the device); only growing a library-owned buffer releases the smaller one.
//   * Calls on one stream from several host threads take the buffer in turn (a per-stream lock held while
//     enqueueing), so their work cannot interleave on it.
//   * On release an event is recorded on the stream, and the next taker's stream waits for it: if a stream is
//     destroyed with work pending and its handle comes back for a new stream, the new work still waits.
//   * A thread holding a StreamWorkspace may not take another (the GEMMs such a call launches get explicit
//     pieces of its buffer); doing so fails with hipErrorInvalidValue instead of deadlocking.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

namespace nnh {

// Offsets of 256-byte-aligned pieces in one buffer.
struct WorkspacePlan {
	size_t total = 0;
	size_t add(size_t bytes) {
		const size_t off = total;
		total += (bytes + 255) & ~static_cast<size_t>(255);
		return off;
	}
};

class StreamWorkspace {
public:
	StreamWorkspace(hipStream_t s, size_t bytes);
	~StreamWorkspace();
	StreamWorkspace(const StreamWorkspace&) = delete;
	StreamWorkspace& operator=(const StreamWorkspace&) = delete;
	hipError_t error() const { return err_; }
	template <typename T>
	T* at(size_t offset) const {
		return reinterpret_cast<T*>(static_cast<char*>(ptr_) + offset);
	}

private:
	void* slot_ = nullptr;
	void* ptr_ = nullptr;
	hipStream_t s_ = nullptr;
	hipError_t err_ = hipSuccess;
};

// Registers the caller's device buffer [p, p + bytes) as stream s's scratch (p null: the library owns it again).
// Waits until no call is enqueueing on s; work already enqueued keeps the buffer it was given.
hipError_t set_stream_workspace(hipStream_t s, void* p, size_t bytes);

// Whether stream s has a caller-registered buffer, and its size.
hipError_t stream_workspace_external(hipStream_t s, bool& external, size_t& bytes);

}  // namespace nnh
