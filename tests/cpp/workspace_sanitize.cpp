// workspace_sanitize.cpp - TEST CODE: nn-cpp_amd/src/workspace_table.hpp (the per-stream scratch slots behind every
// C-ABI call that needs device scratch) run on a host-only stand-in for the HIP runtime, first one step at a time and
// then from many threads at once. Built by tests/cpp/Makefile's `sanitize` target twice, with
// -fsanitize=address,undefined and with -fsanitize=thread, and run by tests/test_sanitize.py on the CPU.
//
// The stand-in: a stream is a device number; stream-ordered allocation and release are malloc and free at once
// (this device finishes every piece of work as it is enqueued, so a buffer released in stream order is gone for
// good the moment free_async returns and any later touch of it is a use after free); events count their
// records. Exit status 0 when every check held; the sanitizers abort on their first report.
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <thread>
#include <vector>

#include "workspace_table.hpp"

namespace {

struct FakeStream {
	int device;
};

struct FakeEvent {
	std::atomic<long> records{0};
};

std::atomic<long> g_allocs{0}, g_frees{0}, g_failed_allocs{0}, g_events{0}, g_waits{0}, g_bad_waits{0};
std::atomic<long> g_fail_every{0};  // > 0: every n-th allocation fails

struct FakeRuntime {
	using Stream = FakeStream*;
	using Event = FakeEvent*;
	using Error = int;
	static constexpr Error kOk = 0;
	static constexpr Error kInvalid = 1;
	static constexpr Error kNoMemory = 2;
	static constexpr Error kNoStream = 3;
	static Error device_of(Stream s, int& dev) {
		if (!s) return kNoStream;
		dev = s->device;
		return kOk;
	}
	static Error malloc_async(void** p, size_t bytes, Stream) {
		const long n = g_allocs.fetch_add(1) + 1;
		const long every = g_fail_every.load();
		if (every > 0 && n % every == 0) {
			g_failed_allocs.fetch_add(1);
			return kNoMemory;
		}
		*p = std::malloc(bytes);
		return *p ? kOk : kNoMemory;
	}
	static Error free_async(void* p, Stream) {
		std::free(p);
		g_frees.fetch_add(1);
		return kOk;
	}
	static Error create_event(Event& ev) {
		ev = new FakeEvent;  // lives as long as its slot, which lives as long as the table
		g_events.fetch_add(1);
		return kOk;
	}
	static Error record_event(Event ev, Stream) {
		ev->records.fetch_add(1);
		return kOk;
	}
	static Error wait_event(Stream, Event ev) {
		g_waits.fetch_add(1);
		if (!ev || ev->records.load() == 0) g_bad_waits.fetch_add(1);  // a wait on an event never recorded
		return kOk;
	}
};

using Table = nnh::WorkspaceTable<FakeRuntime>;

std::atomic<int> g_failures{0};

// Tables live until the process ends, as the library's one does: the list is never destroyed, so their slots and
// buffers stay reachable when the leak checker runs at exit.
std::vector<Table*>* g_tables = new std::vector<Table*>;

Table& new_table() {
	g_tables->push_back(new Table);
	return *g_tables->back();
}

void check(bool ok, const char* what) {
	if (!ok) {
		std::fprintf(stderr, "FAILED: %s\n", what);
		++g_failures;
	}
}

// The same steps as the library's StreamWorkspace: take, use, let go.
struct Take {
	Table& t;
	FakeStream* s;
	void* slot = nullptr;
	void* ptr = nullptr;
	int err;
	Take(Table& table, FakeStream* stream, size_t bytes) : t(table), s(stream) { err = t.acquire(s, bytes, slot, ptr); }
	~Take() { t.release(slot, s); }
};

void single_thread() {
	Table& t = new_table();
	FakeStream s0{0}, s1{1};
	void* first = nullptr;
	{
		Take a(t, &s0, 100);
		check(a.err == FakeRuntime::kOk && a.ptr, "first take succeeds");
		std::memset(a.ptr, 1, 256);  // at least 256 bytes, whatever was asked
		first = a.ptr;
		Take nested(t, &s1, 64);  // a second buffer while holding one
		check(nested.err == FakeRuntime::kInvalid && !nested.slot, "a nested take fails without locking");
		check(t.set_external(&s1, first, 256) == FakeRuntime::kInvalid, "registering while holding fails");
	}
	{
		Take a(t, &s0, 200);
		check(a.ptr == first, "a smaller take reuses the buffer");
	}
	const long frees_before = g_frees.load();
	{
		Take a(t, &s0, 1000);
		check(a.err == FakeRuntime::kOk && a.ptr, "a larger take succeeds");
		std::memset(a.ptr, 2, 1000);
		check(g_frees.load() == frees_before + 1, "growing releases the smaller buffer");
	}
	void* owned = nullptr;
	size_t owned_bytes = 0;
	t.owned(&s0, owned, owned_bytes);
	check(owned_bytes == 1000, "growth takes max(asked, 1.5 x old)");
	{
		Take a(t, &s0, 1100);
		std::memset(a.ptr, 3, 1100);
	}
	t.owned(&s0, owned, owned_bytes);
	check(owned_bytes == 1500, "growth by half the old size");

	// a caller's buffer: handed out as is, never grown; the owned buffer comes back when it is withdrawn
	std::vector<char> ext(512);
	check(t.set_external(&s0, ext.data(), ext.size()) == FakeRuntime::kOk, "register");
	bool is_ext = false;
	size_t ext_bytes = 0;
	t.external(&s0, is_ext, ext_bytes);
	check(is_ext && ext_bytes == 512, "registered buffer reported");
	{
		Take a(t, &s0, 300);
		check(a.err == FakeRuntime::kOk && a.ptr == ext.data(), "the caller's buffer is handed out");
	}
	{
		Take a(t, &s0, 600);
		check(a.err == FakeRuntime::kInvalid && a.slot, "a take beyond the caller's buffer fails (slot still held)");
	}
	check(t.set_external(&s0, nullptr, 0) == FakeRuntime::kOk, "withdraw");
	{
		Take a(t, &s0, 300);
		check(a.ptr == owned, "the library's buffer again");
	}
	{
		Take a(t, nullptr, 64);
		check(a.err == FakeRuntime::kNoStream && !a.slot, "a stream lookup error leaves nothing held");
	}
	// the same stream handle on another device is another slot
	FakeStream moved{5};
	{
		Take a(t, &moved, 64);
		check(a.err == FakeRuntime::kOk && a.ptr != owned, "slots are per (device, stream)");
	}
	check(g_bad_waits.load() == 0, "every wait is on a recorded event");
}

// Many threads on a few streams of two devices: random sizes, a caller's buffer registered and withdrawn on one
// stream meanwhile, allocation failures injected. Each holder fills its whole request with its own byte and checks
// it is still there before letting go: two holders of one buffer would clash (and the thread sanitizer reports
// the race); a buffer shorter than the request or already released is an address sanitizer report.
void many_threads(int threads, int iters, long fail_every) {
	Table& t = new_table();
	std::vector<FakeStream> streams{{0}, {0}, {0}, {1}, {1}, {1}};
	std::vector<char> ext(8192);
	std::atomic<bool> stop{false};
	std::atomic<long> ext_hits{0}, ext_refusals{0}, alloc_errors{0}, nested_tries{0}, nested_ok{0};
	g_fail_every = fail_every;
	const long allocs0 = g_allocs.load(), failed0 = g_failed_allocs.load(), frees0 = g_frees.load();

	std::thread toggler([&] {
		int i = 0;
		while (!stop.load()) {
			const bool on = (i++ & 1) == 0;
			if (t.set_external(&streams[0], on ? ext.data() : nullptr, on ? ext.size() : 0) != FakeRuntime::kOk)
				check(false, "register from a thread holding nothing");
			std::this_thread::yield();
		}
		t.set_external(&streams[0], nullptr, 0);
	});
	std::vector<std::thread> workers;
	for (int w = 0; w < threads; ++w)
		workers.emplace_back([&, w] {
			std::mt19937 rng(1234 + w);
			const unsigned char mark = (unsigned char)(w + 1);
			for (int i = 0; i < iters; ++i) {
				FakeStream* s = &streams[rng() % streams.size()];
				const size_t bytes = 1 + rng() % 16384;
				Take a(t, s, bytes);
				if (a.err == FakeRuntime::kNoMemory) {
					alloc_errors.fetch_add(1);
					continue;
				}
				if (a.err == FakeRuntime::kInvalid) {  // only a registered buffer smaller than the request refuses
					check(s == &streams[0] && bytes > ext.size(), "refusal only for a request beyond the caller's buffer");
					ext_refusals.fetch_add(1);
					continue;
				}
				check(a.err == FakeRuntime::kOk && a.ptr && a.slot, "take");
				if (a.ptr == ext.data()) ext_hits.fetch_add(1);
				unsigned char* p = static_cast<unsigned char*>(a.ptr);
				std::memset(p, mark, bytes);
				if (i % 64 == 0) {
					Take nested(t, &streams[(rng() % 5) + 1], 64);
					nested_tries.fetch_add(1);
					if (nested.err == FakeRuntime::kInvalid && !nested.slot) nested_ok.fetch_add(1);
				}
				std::this_thread::yield();
				bool intact = p[0] == mark && p[bytes / 2] == mark && p[bytes - 1] == mark;
				check(intact, "a buffer is held by one thread at a time");
			}
		});
	for (auto& th : workers) th.join();
	stop = true;
	toggler.join();
	g_fail_every = 0;

	// every successful allocation is either released or still owned by exactly one slot
	long owned_now = 0;
	for (auto& s : streams) {
		void* p = nullptr;
		size_t b = 0;
		t.owned(&s, p, b);
		if (p) ++owned_now;
	}
	const long ok_allocs = (g_allocs.load() - allocs0) - (g_failed_allocs.load() - failed0);
	check(ok_allocs == (g_frees.load() - frees0) + owned_now, "no buffer lost or released twice");
	check(nested_ok.load() == nested_tries.load(), "every nested take is refused");
	check(g_bad_waits.load() == 0, "every wait is on a recorded event");
	std::printf("threads %d x %d takes: %ld caller-buffer takes, %ld refusals, %ld injected allocation failures, "
	            "%ld nested takes refused\n",
	            threads, iters, ext_hits.load(), ext_refusals.load(), alloc_errors.load(), nested_ok.load());
	if (fail_every > 0) check(alloc_errors.load() > 0, "injected failures were seen");
	check(ext_hits.load() > 0, "the caller's buffer was used");
}

}  // namespace

int main(int argc, char** argv) {
	const int iters = argc > 1 ? std::atoi(argv[1]) : 4000;
	single_thread();
	many_threads(8, iters, 0);
	many_threads(8, iters, 2);
	if (g_failures) {
		std::fprintf(stderr, "%d checks failed\n", g_failures.load());
		return 1;
	}
	std::printf("workspace table: all checks passed\n");
	return 0;
}
