// workspace.hip - the per-(device, stream) scratch buffers of workspace.hpp.
#include "workspace.hpp"

#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

namespace nnh {

namespace {

struct Slot {
	std::mutex busy;            // held while a call enqueues work that uses the buffer
	void* owned = nullptr;      // the library's buffer (kept while a caller's buffer is registered)
	size_t owned_bytes = 0;
	void* ext = nullptr;        // the caller's buffer, when one is registered
	size_t ext_bytes = 0;
	hipEvent_t done = nullptr;  // recorded on the stream when the last user let go of the buffer
	bool recorded = false;
};

std::mutex table_mu;
std::map<std::pair<int, hipStream_t>, Slot*> table;  // slots live until the process ends
thread_local bool holding = false;

hipError_t find_slot(hipStream_t s, Slot*& slot) {
	hipDevice_t dev = 0;
	const hipError_t e = hipStreamGetDevice(s, &dev);
	if (e != hipSuccess) return e;
	std::lock_guard<std::mutex> lock(table_mu);
	Slot*& entry = table[{static_cast<int>(dev), s}];
	if (!entry) entry = new Slot;
	slot = entry;
	return hipSuccess;
}

}  // namespace

StreamWorkspace::StreamWorkspace(hipStream_t s, size_t bytes) : s_(s) {
	if (holding) {
		err_ = hipErrorInvalidValue;
		return;
	}
	Slot* slot = nullptr;
	err_ = find_slot(s, slot);
	if (err_ != hipSuccess) return;
	slot->busy.lock();
	slot_ = slot;
	holding = true;
	if (slot->recorded) {  // earlier work that used the buffer (on this stream, or on a destroyed one) comes first
		err_ = hipStreamWaitEvent(s, slot->done, 0);
		if (err_ != hipSuccess) return;
	}
	if (slot->ext) {  // the caller's buffer: never grown here (callers check the size before enqueueing)
		if (bytes > slot->ext_bytes) {
			err_ = hipErrorInvalidValue;
			return;
		}
		ptr_ = slot->ext;
		return;
	}
	bytes = std::max<size_t>(bytes, 256);
	if (slot->owned_bytes < bytes) {
		const size_t grow = std::max(bytes, slot->owned_bytes + slot->owned_bytes / 2);
		void* p = nullptr;
		err_ = hipMallocAsync(&p, grow, s);
		if (err_ != hipSuccess) return;
		if (slot->owned) {
			err_ = hipFreeAsync(slot->owned, s);  // after every earlier use, in stream order
			if (err_ != hipSuccess) {
				(void)hipFreeAsync(p, s);
				return;
			}
		}
		slot->owned = p;
		slot->owned_bytes = grow;
	}
	ptr_ = slot->owned;
}

StreamWorkspace::~StreamWorkspace() {
	Slot* slot = static_cast<Slot*>(slot_);
	if (!slot) return;
	if (!slot->done && hipEventCreateWithFlags(&slot->done, hipEventDisableTiming) != hipSuccess) slot->done = nullptr;
	slot->recorded = slot->done != nullptr && hipEventRecord(slot->done, s_) == hipSuccess;
	holding = false;
	slot->busy.unlock();
}

hipError_t set_stream_workspace(hipStream_t s, void* p, size_t bytes) {
	if (holding) return hipErrorInvalidValue;
	Slot* slot = nullptr;
	const hipError_t e = find_slot(s, slot);
	if (e != hipSuccess) return e;
	std::lock_guard<std::mutex> lock(slot->busy);
	slot->ext = bytes ? p : nullptr;
	slot->ext_bytes = slot->ext ? bytes : 0;
	return hipSuccess;
}

hipError_t stream_workspace_external(hipStream_t s, bool& external, size_t& bytes) {
	Slot* slot = nullptr;
	const hipError_t e = find_slot(s, slot);
	external = false;
	bytes = 0;
	if (e != hipSuccess) return e;
	std::lock_guard<std::mutex> lock(slot->busy);
	external = slot->ext != nullptr;
	bytes = slot->ext_bytes;
	return hipSuccess;
}

}  // namespace nnh
