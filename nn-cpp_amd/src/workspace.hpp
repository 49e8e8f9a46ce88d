// workspace.hpp - device scratch memory for the work one C-ABI call enqueues on a stream (internal to libnnh).
//
// Each (device, stream) pair owns one buffer that the library allocates, grows on demand and keeps until the
// process ends. A call takes it with a StreamWorkspace for as long as it enqueues work; work on one stream runs
// in order, so the next call on that stream may reuse the buffer at once. No call frees memory on its way
// (hipFreeAsync makes the host wait until the stream reaches it, which would keep the host from running ahead
// of the device); only growing the buffer releases the smaller one.
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

}  // namespace nnh
