// workspace.hip - the per-(device, stream) scratch buffers of workspace.hpp: workspace_table.hpp's bookkeeping
// run on the HIP runtime.
#include "workspace.hpp"

#include "workspace_table.hpp"

namespace nnh {

namespace {

struct HipRuntime {
	using Stream = hipStream_t;
	using Event = hipEvent_t;
	using Error = hipError_t;
	static constexpr Error kOk = hipSuccess;
	static constexpr Error kInvalid = hipErrorInvalidValue;
	static Error device_of(Stream s, int& dev) {
		hipDevice_t d = 0;
		const Error e = hipStreamGetDevice(s, &d);
		dev = static_cast<int>(d);
		return e;
	}
	static Error malloc_async(void** p, size_t bytes, Stream s) { return hipMallocAsync(p, bytes, s); }
	static Error free_async(void* p, Stream s) { return hipFreeAsync(p, s); }
	static Error create_event(Event& ev) { return hipEventCreateWithFlags(&ev, hipEventDisableTiming); }
	static Error record_event(Event ev, Stream s) { return hipEventRecord(ev, s); }
	static Error wait_event(Stream s, Event ev) { return hipStreamWaitEvent(s, ev, 0); }
};

using Table = WorkspaceTable<HipRuntime>;

}  // namespace

StreamWorkspace::StreamWorkspace(hipStream_t s, size_t bytes) : s_(s) {
	err_ = Table::instance().acquire(s, bytes, slot_, ptr_);
}

StreamWorkspace::~StreamWorkspace() { Table::instance().release(slot_, s_); }

hipError_t set_stream_workspace(hipStream_t s, void* p, size_t bytes) {
	return Table::instance().set_external(s, p, bytes);
}

hipError_t stream_workspace_external(hipStream_t s, bool& external, size_t& bytes) {
	return Table::instance().external(s, external, bytes);
}

}  // namespace nnh
