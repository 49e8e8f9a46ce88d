// workspace_table.hpp - the bookkeeping behind StreamWorkspace (workspace.hpp): one scratch slot per
// (device, stream), its lock, growth and the caller-registered buffer. It is written over a runtime policy so that
// workspace.hip runs it on HIP and tests/cpp/workspace_sanitize.cpp runs the same code on a host-only stand-in
// under the address, undefined-behaviour and thread sanitizers. No HIP header is needed here.
//
// Rt provides the types Stream, Event and Error, the constants kOk and kInvalid, and
//   Error device_of(Stream, int&)              the device a stream belongs to
//   Error malloc_async(void**, size_t, Stream)  stream-ordered allocation
//   Error free_async(void*, Stream)             stream-ordered release
//   Error create_event(Event&)                  an event without timing
//   Error record_event(Event, Stream)
//   Error wait_event(Stream, Event)             the stream's later work waits for the event
#pragma once

#include <stddef.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

namespace nnh {

template <class Rt>
class WorkspaceTable {
public:
	using Stream = typename Rt::Stream;
	using Event = typename Rt::Event;
	using Error = typename Rt::Error;

	// The table of the process: never destroyed, so no slot is freed while static destructors run.
	static WorkspaceTable& instance() {
		static WorkspaceTable* table = new WorkspaceTable;
		return *table;
	}

	// Takes stream s's slot for a call needing `bytes` of scratch. On return `slot` is set whenever the slot's lock
	// was taken (also when an error follows); the caller then calls release(slot, s) exactly once. `ptr` is the
	// buffer when the result is kOk.
	Error acquire(Stream s, size_t bytes, void*& slot, void*& ptr) {
		slot = nullptr;
		ptr = nullptr;
		if (holding()) return Rt::kInvalid;  // one thread, one buffer: a nested take would deadlock
		Slot* sl = nullptr;
		Error e = find(s, sl);
		if (e != Rt::kOk) return e;
		sl->busy.lock();
		slot = sl;
		holding() = true;
		if (sl->recorded) {  // earlier work that used the buffer (on this stream, or on a destroyed one) comes first
			e = Rt::wait_event(s, sl->done);
			if (e != Rt::kOk) return e;
		}
		if (sl->ext) {  // the caller's buffer: never grown here (callers check the size before enqueueing)
			if (bytes > sl->ext_bytes) return Rt::kInvalid;
			ptr = sl->ext;
			return Rt::kOk;
		}
		bytes = std::max<size_t>(bytes, 256);
		if (sl->owned_bytes < bytes) {
			const size_t grow = std::max(bytes, sl->owned_bytes + sl->owned_bytes / 2);
			void* p = nullptr;
			e = Rt::malloc_async(&p, grow, s);
			if (e != Rt::kOk) return e;
			if (sl->owned) {
				e = Rt::free_async(sl->owned, s);  // after every earlier use, in stream order
				if (e != Rt::kOk) {
					(void)Rt::free_async(p, s);
					return e;
				}
			}
			sl->owned = p;
			sl->owned_bytes = grow;
		}
		ptr = sl->owned;
		return Rt::kOk;
	}

	// Lets go of a slot acquire() took: records the slot's event on s, so the next taker's stream waits for this
	// call's work, and unlocks it.
	void release(void* slot, Stream s) {
		Slot* sl = static_cast<Slot*>(slot);
		if (!sl) return;
		if (!sl->has_event) sl->has_event = Rt::create_event(sl->done) == Rt::kOk;
		sl->recorded = sl->has_event && Rt::record_event(sl->done, s) == Rt::kOk;
		holding() = false;
		sl->busy.unlock();
	}

	// Registers [p, p + bytes) as stream s's scratch (p null or bytes 0: the library's own buffer again). Waits
	// until no call is enqueueing on s.
	Error set_external(Stream s, void* p, size_t bytes) {
		if (holding()) return Rt::kInvalid;
		Slot* sl = nullptr;
		const Error e = find(s, sl);
		if (e != Rt::kOk) return e;
		std::lock_guard<std::mutex> lock(sl->busy);
		sl->ext = bytes ? p : nullptr;
		sl->ext_bytes = sl->ext ? bytes : 0;
		return Rt::kOk;
	}

	// Whether stream s has a registered buffer, and its size.
	Error external(Stream s, bool& ext, size_t& bytes) {
		ext = false;
		bytes = 0;
		Slot* sl = nullptr;
		const Error e = find(s, sl);
		if (e != Rt::kOk) return e;
		std::lock_guard<std::mutex> lock(sl->busy);
		ext = sl->ext != nullptr;
		bytes = sl->ext_bytes;
		return Rt::kOk;
	}

	// The library-owned buffer of stream s and its size (null, 0 before the first take): for tests.
	Error owned(Stream s, void*& p, size_t& bytes) {
		p = nullptr;
		bytes = 0;
		Slot* sl = nullptr;
		const Error e = find(s, sl);
		if (e != Rt::kOk) return e;
		std::lock_guard<std::mutex> lock(sl->busy);
		p = sl->owned;
		bytes = sl->owned_bytes;
		return Rt::kOk;
	}

private:
	struct Slot {
		std::mutex busy;          // held while a call enqueues work that uses the buffer
		void* owned = nullptr;    // the library's buffer (kept while a caller's buffer is registered)
		size_t owned_bytes = 0;
		void* ext = nullptr;      // the caller's buffer, when one is registered
		size_t ext_bytes = 0;
		Event done{};             // recorded on the stream when the last user let go of the buffer
		bool has_event = false;
		bool recorded = false;
	};

	static bool& holding() {
		static thread_local bool held = false;
		return held;
	}

	Error find(Stream s, Slot*& slot) {
		int dev = 0;
		const Error e = Rt::device_of(s, dev);
		if (e != Rt::kOk) return e;
		std::lock_guard<std::mutex> lock(mu_);
		Slot*& entry = table_[{dev, s}];
		if (!entry) entry = new Slot;  // slots live as long as the table
		slot = entry;
		return Rt::kOk;
	}

	std::mutex mu_;
	std::map<std::pair<int, Stream>, Slot*> table_;
};

}  // namespace nnh
