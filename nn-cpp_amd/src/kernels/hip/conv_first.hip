// conv_first.hip - the whole backward of a network's first convolution layer (K = Cin*kh*kw <= 16, at most 32
// output channels, stride 1) in one workgroup per sample (src/autograd/ops.cpp:1418-1463).
//
// The reference computes, per sample n, the masked gradient g' = alive ? g : 0 (ops.cpp:1439-1443), db_n[co] =
// lane_sum(g'[co]) (1445), dW_n = g' col_n^T (1448-1449: each dW_n[co][k] the fma chain over the output positions p
// in order from +0 of g'[co][p] col_n[k][p]) and dx = col2im(W^T g') (1452-1455: each dcol[k][p] the fma chain over
// co in order from +0 of W[co][k] g'[co][p]; each dx element then adds its taps in (ph, pw) order, starting from 0 or
// its old value). The caller sums db_n and dW_n over the samples in order.
//
// A workgroup of twelve waves walks the sample's output positions in chunks of 128, one barrier per chunk, with each
// wave in one role:
//   * waves 4-11 stream the gradient from HBM (kFbRing chunks of loads in flight), mask it and write each chunk into
//     one of two LDS slots, transposed by 16 positions (position 16 J + 4 t + e at 16 J + 4 e + t, so that one 16-byte
//     read feeds four MFMA steps), together with the chunk's im2col columns taken from the input plane in LDS;
//   * waves 0-1 run dW_n and db_n for 16 channels each as one 16x16x4 MFMA chain (four fmas in sequence per element
//     and instruction, bit for bit): at step 4 J + t lane (grp, c) supplies g'[c][16 J + 4 t + grp] and lane (grp, k)
//     col[k][the same position]; lane_sum's partials ride along (position 16 J + 4 t + grp is partial grp for even t,
//     grp + 4 for odd t). These waves do little besides LDS reads and the chain: a dependent MFMA does not overlap
//     VALU work of its own wave, so such work would lengthen every step. Steps past hw multiply +0 by -0, which
//     changes no sum;
//   * waves 2-3 compute dcol for the chunk's positions as 16x16x4 chains over the output channels (A: g' from the
//     slot, B: W in registers) into an LDS buffer for the whole plane;
//   * after the last chunk every wave gathers dx: each element adds its taps in (ph, pw) order.
#include "conv.hpp"

#include <algorithm>

#include "fastdiv.hpp"
#include "gemm.hpp"
#include "gemm_tile.hpp"

namespace nnh {

namespace {

constexpr int kFbThreads = 768;
constexpr int kFbMaxK = 16;
constexpr int kFbMaxCo = 32;
constexpr int kFbChunk = 128;              // output positions per chunk (eight blocks of 16)
constexpr int kFbBlocks = kFbChunk / 16;
constexpr int kFbRowQuads = kFbChunk / 4;  // quads of a gradient row in a chunk
constexpr int kFbPitch = kFbChunk + 4;     // LDS pitch of a row of a chunk slot
constexpr int kFbSlot = 48 * kFbPitch;     // 32 gradient rows and 16 column rows
constexpr int kFbRing = 6;                 // chunks of gradient loads in flight per staging lane
constexpr int kFbMaxPlane = 2048;
constexpr size_t kFbMaxLds = 160 * 1024;
// staging lanes (waves 4 on): each builds kFbQuads gradient quads and kFbCols column values of every chunk. Eight
// staging waves keep a chunk's build (masking, the transposed LDS writes, the im2col gathers) about as long as the
// dW chain's 16 MFMAs, which four waves were not.
constexpr int kFbStage = kFbThreads - 256;
constexpr int kFbQuads = 32 * kFbChunk / 4 / kFbStage;
constexpr int kFbCols = 16 * kFbChunk / kFbStage;
static_assert(kFbQuads * kFbStage == 32 * kFbChunk / 4 && kFbCols * kFbStage == 16 * kFbChunk &&
                  kFbStage % kFbChunk == 0 && kFbChunk % 64 == 0 && kFbStage % kFbRowQuads == 0,
              "whole quads and columns per staging lane, a column's positions within one wave pair");

// flag layouts: none, one byte per position (a 4-byte word per quad of positions), or one bit per position (bit o of
// the flattened output index at byte o / 8, bit o % 8: a quad's flags are one nibble)
constexpr int kAlNone = 0, kAlWord = 1, kAlBits = 2;

struct FbArgs {
	const float* g;               // output gradient {N, Cout, hw}
	const unsigned char* alive;   // the forward's ReLU flags (read only by the instantiations that mask)
	const float* x;               // {N, Cin, H, W}
	const float* w;               // {Cout, K}
	float* gb;                    // per-sample bias sums {N, Cout}, or null
	float* gw;                    // per-sample weight gradients {N, Cout, K}
	float* dx;                    // {N, Cin, H, W}, or null
	int dx_first;
	ConvGeom geo;
	int cout, K, hw, full, nchunks;
	int hp, wp, plane, plane_pad; // zero-padded input plane: (ho-1) + kh rows, (wo-1) + kw columns
	int dpitch;                   // LDS pitch of a dcol row (nchunks * kFbChunk + 4)
	int koff[kFbMaxK];            // column k = (ci, ph, pw) starts at plane offset (ci hp + ph) wp + pw (0 past K)
	int tapc[kFbMaxK];            // tap t = (ph, pw): t dpitch - ph wo - pw (0 past kh kw)
	FastDiv wo_div, plane_div, wp_div, w_div;
};

__device__ __forceinline__ int fb_slot(int p) { return (p & ~15) + 4 * (p & 3) + ((p >> 2) & 3); }

// KM: K <= KM (9 or 16) taps per input channel; NS: 4 or 8 steps of four output channels in a dcol chain
// (Cout <= 4 NS); AL: the flag layout.
template <int KM, int NS, int AL>
__global__ void __launch_bounds__(kFbThreads) conv_first_bwd_kernel(const FbArgs a) {
	extern __shared__ __align__(16) float sm[];
	const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
	const ConvGeom& G = a.geo;
	const int hw = a.hw, K = a.K, full = a.full, nchunks = a.nchunks;
	const int n = blockIdx.x;
	const int64_t row0 = (int64_t)n * a.cout;
	float* slots = sm;                          // two chunk slots
	float* plane = sm + 2 * kFbSlot;            // the zero-padded input plane
	float* dcb = plane + a.plane_pad;           // [K + 1][dpitch]: dcol (row K takes the lanes past K)

	// Every wave passes 2 + nchunks barriers below (and one more when dx is asked for), whatever its role.
	if (wave >= 4) {
		// ---- staging: lane st owns quads st + kFbStage u of each chunk (row = quad / kFbRowQuads, positions
		// 4 (quad % kFbRowQuads) ..)
		const int st = tid - 256;
		// the columns this lane builds: value st + kFbStage u of a chunk is column (st + kFbStage u) / kFbChunk =
		// kcol0 + kFbStage / kFbChunk u (wave-uniform) at position st % kFbChunk, the same in every chunk. Their plane
		// offsets are read once with a wave-uniform index: a per-lane index into the argument block becomes a vector
		// load whose wait would also drain the ring of gradient loads in flight
		const int kcol0 = (wave - 4) * 64 / kFbChunk, pcol = st & (kFbChunk - 1);
		int koff[kFbCols];
#pragma unroll
		for (int u = 0; u < kFbCols; ++u) koff[u] = a.koff[min(kcol0 + kFbStage / kFbChunk * u, K - 1)];
		// a lane's quads keep their rows (st / kFbRowQuads + kFbStage / kFbRowQuads u) and their place in the chunk
		// (4 (st % kFbRowQuads)) in every chunk: the row offsets and the rows' liveness once
		const int q4 = 4 * (st % kFbRowQuads);
		int64_t roff[kFbQuads];
		bool rlive[kFbQuads];
#pragma unroll
		for (int u = 0; u < kFbQuads; ++u) {
			const int row = st / kFbRowQuads + kFbStage / kFbRowQuads * u;
			rlive[u] = row < a.cout;
			roff[u] = (row0 + min(row, a.cout - 1)) * hw;
		}
		auto load = [&](int ch, f32x4(&v)[kFbQuads], unsigned(&f)[kFbQuads]) {
#pragma unroll
			for (int u = 0; u < kFbQuads; ++u) {
				const int p = min(ch * kFbChunk + q4, hw - 4);
				const int64_t at = roff[u] + p;
				v[u] = *reinterpret_cast<const f32x4*>(a.g + at);
				if (AL == kAlWord) {
					f[u] = *reinterpret_cast<const unsigned*>(a.alive + at);
				} else if (AL == kAlBits) {
					// the quad's nibble spread to one flag byte per position
					const unsigned nb = (unsigned)(a.alive[at >> 3] >> (at & 4)) & 0xfu;
					f[u] = (nb & 1u) | ((nb & 2u) << 7) | ((nb & 4u) << 14) | ((nb & 8u) << 21);
				} else {
					f[u] = 0x01010101u;
				}
			}
		};
		// chunk ch into slot ch % 2: the masked gradient (rows past cout and positions past hw are zero) and the
		// columns
		auto build = [&](int ch, const f32x4(&v)[kFbQuads], const unsigned(&f)[kFbQuads]) {
			float* sl = slots + (ch & 1) * kFbSlot;
#pragma unroll
			for (int u = 0; u < kFbQuads; ++u) {
				const int qi = st + kFbStage * u, row = qi / kFbRowQuads, q = qi % kFbRowQuads;
				// hw is a multiple of 4, so a quad lies wholly before hw or wholly past it
				const bool on = rlive[u] && ch * kFbChunk + q4 < hw;
				float* d = sl + row * kFbPitch + 16 * (q >> 2) + (q & 3);
#pragma unroll
				for (int e = 0; e < 4; ++e) d[4 * e] = (on && ((f[u] >> (8 * e)) & 0xffu)) ? v[u][e] : 0.0f;
			}
			// the columns' values at position ch * kFbChunk + pcol; all reads are issued before the writes
			float cv[kFbCols];
			const unsigned pq = (unsigned)min(ch * kFbChunk + pcol, hw - 1);
			const int oh = (int)fdiv(pq, a.wo_div), ow = (int)pq - oh * G.wo;
#pragma unroll
			for (int u = 0; u < kFbCols; ++u) cv[u] = plane[koff[u] + oh * a.wp + ow];
#pragma unroll
			for (int u = 0; u < kFbCols; ++u) {
				const int k = kcol0 + kFbStage / kFbChunk * u;
				if (k < K) sl[(32 + k) * kFbPitch + fb_slot(pcol)] = ch * kFbChunk + pcol < hw ? cv[u] : 0.0f;
			}
		};
		f32x4 rv[kFbRing][kFbQuads];
		unsigned rf[kFbRing][kFbQuads];
#pragma unroll
		for (int u = 0; u < kFbRing; ++u) load(u, rv[u], rf[u]);
		__syncthreads();  // the plane is in LDS
		build(0, rv[0], rf[0]);
		load(kFbRing, rv[0], rf[0]);
		__syncthreads();  // chunk 0 is in slot 0
		// iteration i builds chunk i + 1 (i < nchunks - 1) while the other waves work on chunk i; whole trips of the
		// ring keep the waits exact
		const int last = nchunks - 1;
		const int trips = last / kFbRing;
		for (int tr = 0; tr < trips; ++tr) {
#pragma unroll
			for (int u = 0; u < kFbRing; ++u) {
				const int i = tr * kFbRing + u;
				build(i + 1, rv[(u + 1) % kFbRing], rf[(u + 1) % kFbRing]);
				load(i + 1 + kFbRing, rv[(u + 1) % kFbRing], rf[(u + 1) % kFbRing]);
				__syncthreads();
			}
		}
		// the remaining iterations trips * kFbRing .. nchunks - 1 (at most kFbRing of them)
#pragma unroll
		for (int u = 0; u < kFbRing; ++u) {
			const int i = trips * kFbRing + u;
			if (i < last) build(i + 1, rv[(u + 1) % kFbRing], rf[(u + 1) % kFbRing]);
			if (i < nchunks) __syncthreads();
		}
	} else {
		// ---- waves 0-3: the input plane first (plane[ci][r][q] = x[ci][r - pad][q - pad], 0 outside)
		const float* xn = a.x + (int64_t)n * G.cin * G.h * G.w;
		float xv[kFbMaxPlane / 256];
#pragma unroll
		for (int u = 0; u < kFbMaxPlane / 256; ++u) {
			const int e = min(tid + 256 * u, a.plane - 1);
			const int ci = (int)fdiv((unsigned)e, a.plane_div), rem = e - ci * (a.hp * a.wp);
			const int r = (int)fdiv((unsigned)rem, a.wp_div), q = rem - r * a.wp;
			const int ih = min(max(r - G.pad, 0), G.h - 1), iw = min(max(q - G.pad, 0), G.w - 1);
			xv[u] = xn[((int64_t)ci * G.h + ih) * G.w + iw];
		}
#pragma unroll
		for (int u = 0; u < kFbMaxPlane / 256; ++u) {
			const int e = tid + 256 * u;
			if (e < a.plane) {
				const int ci = (int)fdiv((unsigned)e, a.plane_div), rem = e - ci * (a.hp * a.wp);
				const int r = (int)fdiv((unsigned)rem, a.wp_div), q = rem - r * a.wp;
				const int ih = r - G.pad, iw = q - G.pad;
				plane[e] = (ih >= 0 && ih < G.h && iw >= 0 && iw < G.w) ? xv[u] : 0.0f;
			}
		}
		__syncthreads();  // the plane is in LDS
		__syncthreads();  // chunk 0 is in slot 0
		const int grp = lane >> 4, l16 = lane & 15;
		if (wave < 2) {
			// ---- dW_n and db_n for channels c0 .. c0 + 15 (lane (grp, c): row c0 + c; lane (grp, k): column k)
			const int c0 = 16 * wave, c = l16, k = l16;
			const bool live = c0 < a.cout;
			f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
			float part0 = 0.0f, part1 = 0.0f;
			const int arow = min(c0 + c, 31) * kFbPitch + 4 * grp;        // rows past cout are zero
			const int brow = (32 + min(k, K - 1)) * kFbPitch + 4 * grp;   // columns past K: never stored
			for (int i = 0; i < nchunks; ++i) {
				if (live) {
					const float* sl = slots + (i & 1) * kFbSlot;
					f32x4 av[kFbBlocks], bv[kFbBlocks];
#pragma unroll
					for (int b = 0; b < kFbBlocks; ++b) {
						av[b] = *reinterpret_cast<const f32x4*>(sl + arow + 16 * b);
						bv[b] = *reinterpret_cast<const f32x4*>(sl + brow + 16 * b);
					}
					if ((i + 1) * kFbChunk <= full) {
#pragma unroll
						for (int b = 0; b < kFbBlocks; ++b)
#pragma unroll
							for (int t = 0; t < 4; ++t) {
								if (t & 1) part1 = part1 + av[b][t];
								else part0 = part0 + av[b][t];
								acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[b][t], bv[b][t], acc, 0, 0, 0);
							}
					} else {
						// the chunk reaches past full: positions past hw multiply +0 by -0, past full skip the partials
#pragma unroll
						for (int b = 0; b < kFbBlocks; ++b)
#pragma unroll
							for (int t = 0; t < 4; ++t) {
								const int p = i * kFbChunk + 16 * b + 4 * t + grp;
								const float b_t = p < hw ? bv[b][t] : -0.0f;
								if (t & 1) part1 = p < full ? part1 + av[b][t] : part1;
								else part0 = p < full ? part0 + av[b][t] : part0;
								acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[b][t], b_t, acc, 0, 0, 0);
							}
					}
				}
				__syncthreads();
			}
			// dW_n[c0 + 4 grp + r][k] sits in register r of lane (grp, k)
			float* gwn = a.gw + (row0 + c0) * K;
			if (live && k < K) {
#pragma unroll
				for (int r = 0; r < 4; ++r)
					if (c0 + 4 * grp + r < a.cout) gwn[(int64_t)(4 * grp + r) * K + k] = acc[r];
			}
			if (live && a.gb) {
				// lane_sum (ops.cpp:804-812): partials a0..a3 are part0 of lanes c, c + 16, c + 32, c + 48 and a4..a7
				// their part1; ((a0 + a1) + (a2 + a3)) + ((a4 + a5) + (a6 + a7)), then the tail (positions full ..
				// hw - 1, all in the last chunk's slot) in order
				float q[8];
#pragma unroll
				for (int j = 0; j < 4; ++j) {
					q[j] = __shfl(part0, c + 16 * j);
					q[4 + j] = __shfl(part1, c + 16 * j);
				}
				if (grp == 0 && c0 + c < a.cout) {
					float s = ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
					const float* sl = slots + ((nchunks - 1) & 1) * kFbSlot + (c0 + c) * kFbPitch;
					for (int p = full; p < hw; ++p) s = s + sl[fb_slot(p - (nchunks - 1) * kFbChunk)];
					a.gb[row0 + c0 + c] = s;
				}
			}
		} else {
			// ---- dcol of the chunk's blocks b0 + 2 j (b0 = wave - 2): lane (grp, i) supplies g'[4 t + grp][16 b +
			// i], lane (grp, j) W[4 t + grp][j]; D[4 grp + r][j] = dcol[j][16 b + 4 grp + r]. Chains over co from +0;
			// steps past cout multiply +0 (the zero rows) by -0.
			const int b0 = wave - 2, i16 = l16;
			float wreg[NS];
#pragma unroll
			for (int t = 0; t < NS; ++t) {
				const int co = 4 * t + grp;
				wreg[t] = (a.dx && co < a.cout && i16 < K) ? a.w[(int64_t)co * K + i16] : -0.0f;
			}
			float* drow = dcb + min(i16, K) * a.dpitch;
			constexpr int kJ = kFbBlocks / 2;
			int sidx[kJ];
#pragma unroll
			for (int j = 0; j < kJ; ++j) sidx[j] = fb_slot(16 * (b0 + 2 * j) + i16);
			for (int i = 0; i < nchunks; ++i) {
				if (a.dx) {
					const float* sl = slots + (i & 1) * kFbSlot + grp * kFbPitch;
					float vv[kJ][NS];
#pragma unroll
					for (int j = 0; j < kJ; ++j)
#pragma unroll
						for (int t = 0; t < NS; ++t) vv[j][t] = sl[4 * t * kFbPitch + sidx[j]];
					f32x4 acc[kJ];
#pragma unroll
					for (int j = 0; j < kJ; ++j) acc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
					for (int t = 0; t < NS; ++t)
#pragma unroll
						for (int j = 0; j < kJ; ++j)
							acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[j][t], wreg[t], acc[j], 0, 0, 0);
#pragma unroll
					for (int j = 0; j < kJ; ++j)
#pragma unroll
						for (int r = 0; r < 4; ++r) drow[i * kFbChunk + 16 * (b0 + 2 * j) + 4 * grp + r] = acc[j][r];
				}
				__syncthreads();
			}
		}
	}
	if (!a.dx) return;
	__syncthreads();  // dcol is complete
	// ---- dx: every element adds its valid taps in (ph, pw) order (col2im_fast_kernel's order), starting from 0 or its
	// old value. Tap t = ph kw + pw is valid when bit t of vmask is set; all KM reads are issued (invalid ones at offset
	// 0) before the adds.
	const int T = G.kh * G.kw, hwi = G.h * G.w, total = G.cin * hwi;
	float* dxn = a.dx + (int64_t)n * total;
	for (int e0 = 0; e0 < total; e0 += kFbThreads) {
		const int e = min(e0 + tid, total - 1);
		const int ci = e / hwi, rem = e - ci * hwi;
		const int ih = (int)fdiv((unsigned)rem, a.w_div), iw = rem - ih * G.w;
		const float old = a.dx_first ? 0.0f : dxn[e];
		const int hlo = max(0, ih + G.pad - G.ho + 1), hhi = min(G.kh - 1, ih + G.pad);
		const int wlo = max(0, iw + G.pad - G.wo + 1), whi = min(G.kw - 1, iw + G.pad);
		const unsigned rows = hhi >= hlo ? (2u << hhi) - (1u << hlo) : 0u;
		const unsigned cols = whi >= wlo ? (2u << whi) - (1u << wlo) : 0u;
		unsigned vmask = 0;
		for (int ph = 0; ph < G.kh; ++ph) vmask |= ((rows >> ph) & 1u) ? cols << (ph * G.kw) : 0u;
		const int base = ci * T * a.dpitch + (ih + G.pad) * G.wo + iw + G.pad;
		float tv[KM];
#pragma unroll
		for (int t = 0; t < KM; ++t) tv[t] = dcb[((vmask >> t) & 1u) ? base + a.tapc[t] : 0];
		float v = old;
#pragma unroll
		for (int t = 0; t < KM; ++t) v = ((vmask >> t) & 1u) ? v + tv[t] : v;
		if (e0 + tid < total) dxn[e] = v;
	}
}

struct FbLayout {
	int hw, K, nchunks, hp, wp, plane, plane_pad, dpitch;
	size_t floats;
};

FbLayout fb_layout(const ConvGeom& g, bool dx) {
	FbLayout l{};
	l.hw = g.ho * g.wo;
	l.K = g.cin * g.kh * g.kw;
	l.nchunks = (l.hw + kFbChunk - 1) / kFbChunk;
	l.hp = g.ho - 1 + g.kh;
	l.wp = g.wo - 1 + g.kw;
	l.plane = g.cin * l.hp * l.wp;
	l.plane_pad = (l.plane + 3) / 4 * 4;
	// four floats past the chunks: a pitch that is a multiple of the 64 banks would put a dcol write's sixteen rows in
	// one bank
	l.dpitch = l.nchunks * kFbChunk + 4;
	l.floats = 2 * (size_t)kFbSlot + (size_t)l.plane_pad + (dx ? (size_t)(l.K + 1) * l.dpitch : 0);
	return l;
}

}  // namespace

bool conv_first_bwd_ok(const ConvGeom& g, int64_t samples, int cout, bool dx, const float* gr,
                       const unsigned char* alive, bool alive_bits) {
	if (alive_bits) alive = nullptr;  // bits take any alignment
	const int64_t hw = (int64_t)g.ho * g.wo, K = (int64_t)g.cin * g.kh * g.kw;
	if (cout < 1 || cout > kFbMaxCo || samples < 1 || samples > 0x7fffffff || hw < 1 || K < 1 || K > kFbMaxK)
		return false;
	// the staging loads 16-byte quads of the gradient and 4-byte words of flags
	if (hw % 4 != 0 || reinterpret_cast<uintptr_t>(gr) % 16 != 0 || reinterpret_cast<uintptr_t>(alive) % 4 != 0)
		return false;
	if (g.stride != 1 || g.h < 1 || g.w < 1 || hw > (1 << 16)) return false;
	const FbLayout l = fb_layout(g, dx);
	if (l.plane > kFbMaxPlane || l.floats * sizeof(float) > kFbMaxLds) return false;
	// the reference's dW_n product sgemm(F, T, Cout, K, hw) and dcol product sgemm(T, F, K, hw, Cout) are single
	// chains per element only without a depth cut (in either numerics mode)
	return !depth_cut(cout, K, hw) && !depth_cut(K, hw, cout);
}

hipError_t conv_first_bwd(const float* g, const unsigned char* alive, const float* x, const float* w, float* gb,
                          float* gw, float* dx, int dx_first, const ConvGeom& geo, int64_t samples, int cout,
                          hipStream_t s, bool alive_bits) {
	if (!conv_first_bwd_ok(geo, samples, cout, dx != nullptr, g, alive, alive_bits)) return hipErrorInvalidValue;
	const FbLayout l = fb_layout(geo, dx != nullptr);
	FbArgs a{};
	a.g = g;
	a.alive = alive;
	a.x = x;
	a.w = w;
	a.gb = gb;
	a.gw = gw;
	a.dx = dx;
	a.dx_first = dx_first;
	a.geo = geo;
	a.cout = cout;
	a.K = l.K;
	a.hw = l.hw;
	a.full = l.hw & ~7;
	a.nchunks = l.nchunks;
	a.hp = l.hp;
	a.wp = l.wp;
	a.plane = l.plane;
	a.plane_pad = l.plane_pad;
	a.dpitch = l.dpitch;
	for (int ci = 0, k = 0; ci < geo.cin; ++ci)
		for (int ph = 0; ph < geo.kh; ++ph)
			for (int pw = 0; pw < geo.kw; ++pw) a.koff[k++] = (ci * a.hp + ph) * a.wp + pw;
	for (int ph = 0, t = 0; ph < geo.kh; ++ph)
		for (int pw = 0; pw < geo.kw; ++pw, ++t) a.tapc[t] = t * a.dpitch - ph * geo.wo - pw;
	a.wo_div = make_fastdiv((unsigned)geo.wo);
	a.plane_div = make_fastdiv((unsigned)(a.hp * a.wp));
	a.wp_div = make_fastdiv((unsigned)a.wp);
	a.w_div = make_fastdiv((unsigned)geo.w);
	using Kern = void (*)(FbArgs);
	static const Kern kerns[2][2][3] = {
	    {{conv_first_bwd_kernel<9, 4, kAlNone>, conv_first_bwd_kernel<9, 4, kAlWord>, conv_first_bwd_kernel<9, 4, kAlBits>},
	     {conv_first_bwd_kernel<9, 8, kAlNone>, conv_first_bwd_kernel<9, 8, kAlWord>, conv_first_bwd_kernel<9, 8, kAlBits>}},
	    {{conv_first_bwd_kernel<16, 4, kAlNone>, conv_first_bwd_kernel<16, 4, kAlWord>,
	      conv_first_bwd_kernel<16, 4, kAlBits>},
	     {conv_first_bwd_kernel<16, 8, kAlNone>, conv_first_bwd_kernel<16, 8, kAlWord>,
	      conv_first_bwd_kernel<16, 8, kAlBits>}}};
	const Kern k = kerns[a.K > 9][cout > 16][alive == nullptr ? 0 : alive_bits ? 2 : 1];
	const size_t lds = l.floats * sizeof(float);
	hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
	                                   (int)lds);
	if (e != hipSuccess) return e;
	hipLaunchKernelGGL(k, dim3((unsigned)samples), dim3(kFbThreads), lds, s, a);
	return hipGetLastError();
}

}  // namespace nnh
