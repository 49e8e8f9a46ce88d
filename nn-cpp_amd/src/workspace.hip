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
	void* p = nullptr;
	size_t bytes = 0;
	hipEvent_t done = nullptr;  // recorded on the stream when the last user let go of the buffer
	bool recorded = false;
};

std::mutex table_mu;
std::map<std::pair<int, hipStream_t>, Slot*> table;  // slots live until the process ends
thread_local bool holding = false;

}  // namespace

StreamWorkspace::StreamWorkspace(hipStream_t s, size_t bytes) : s_(s) {
	if (holding) {
		err_ = hipErrorInvalidValue;
		return;
	}
	hipDevice_t dev = 0;
	err_ = hipStreamGetDevice(s, &dev);
	if (err_ != hipSuccess) return;
	Slot* slot = nullptr;
	{
		std::lock_guard<std::mutex> lock(table_mu);
		Slot*& e = table[{static_cast<int>(dev), s}];
		if (!e) e = new Slot;
		slot = e;
	}
	slot->busy.lock();
	slot_ = slot;
	holding = true;
	if (slot->recorded) {  // earlier work that used the buffer (on this stream, or on a destroyed one) comes first
		err_ = hipStreamWaitEvent(s, slot->done, 0);
		if (err_ != hipSuccess) return;
	}
	bytes = std::max<size_t>(bytes, 256);
	if (slot->bytes < bytes) {
		const size_t grow = std::max(bytes, slot->bytes + slot->bytes / 2);
		void* p = nullptr;
		err_ = hipMallocAsync(&p, grow, s);
		if (err_ != hipSuccess) return;
		if (slot->p) {
			err_ = hipFreeAsync(slot->p, s);  // after every earlier use, in stream order
			if (err_ != hipSuccess) {
				(void)hipFreeAsync(p, s);
				return;
			}
		}
		slot->p = p;
		slot->bytes = grow;
	}
	ptr_ = slot->p;
}

StreamWorkspace::~StreamWorkspace() {
	Slot* slot = static_cast<Slot*>(slot_);
	if (!slot) return;
	if (!slot->done && hipEventCreateWithFlags(&slot->done, hipEventDisableTiming) != hipSuccess) slot->done = nullptr;
	slot->recorded = slot->done != nullptr && hipEventRecord(slot->done, s_) == hipSuccess;
	holding = false;
	slot->busy.unlock();
}

}  // namespace nnh
