// ops_elem.hip - extern "C" entry points of nn::add (broadcast right operand), nn::gelu and nn::embedding
// (include/nnh.h).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "abi_common.hpp"
#include "kernels/hip/elementwise.hpp"
#include "nnh.h"

using namespace nnh;

extern "C" {

int nnh_add_forward(const float* a, const float* b, size_t outer, size_t inner, float* y, void* stream) {
	uint64_t total = 0;
	if (!count_ok({outer, inner}, total)) return fail(NNH_ERR_INVALID, "add: size out of range (above 2^60 elements)");
	if (total == 0) return NNH_OK;
	if (!a || !b || !y) return fail(NNH_ERR_INVALID, "add: null pointer");
	// y may be a itself (element by element), never a partial overlap of a, nor any overlap of b
	if (partial_overlap(y, total * 4, a, total * 4) || ranges_overlap(y, total * 4, b, (uint64_t)inner * 4))
		return fail(NNH_ERR_ALIAS, "add: y overlaps b or part of a");
	return hip_status(add_bcast(a, b, (int64_t)outer, (int64_t)inner, y, reinterpret_cast<hipStream_t>(stream)), "add");
}

int nnh_mul_forward(const float* a, const float* b, size_t count, float* y, void* stream) {
	if (!count_ok({count})) return fail(NNH_ERR_INVALID, "mul: size out of range (above 2^60 elements)");
	if (count == 0) return NNH_OK;
	if (!a || !b || !y) return fail(NNH_ERR_INVALID, "mul: null pointer");
	const uint64_t n = (uint64_t)count * 4;
	// y may be a or b itself (element by element), never a partial overlap of either
	if (partial_overlap(y, n, a, n) || partial_overlap(y, n, b, n)) return fail(NNH_ERR_ALIAS, "mul: y overlaps part of a or b");
	return hip_status(mul(a, b, (int64_t)count, y, reinterpret_cast<hipStream_t>(stream)), "mul");
}

int nnh_mul_backward(const float* g, const float* other, size_t count, float* d, int first, void* stream) {
	if (!count_ok({count})) return fail(NNH_ERR_INVALID, "mul backward: size out of range (above 2^60 elements)");
	if (count == 0) return NNH_OK;
	if (!g || !other || !d) return fail(NNH_ERR_INVALID, "mul backward: null pointer");
	const uint64_t n = (uint64_t)count * 4;
	if (ranges_overlap(d, n, other, n) || partial_overlap(d, n, g, n))
		return fail(NNH_ERR_ALIAS, "mul backward: d overlaps the other operand or part of g");
	return hip_status(mul_grad(g, other, (int64_t)count, d, first ? 1 : 0, reinterpret_cast<hipStream_t>(stream)),
	                  "mul backward");
}

int nnh_gelu_forward(const float* x, size_t count, float* y, float* tanh_saved, void* stream) {
	if (!count_ok({count})) return fail(NNH_ERR_INVALID, "gelu: size out of range (above 2^60 elements)");
	if (count == 0) return NNH_OK;
	if (!x || !y || !tanh_saved) return fail(NNH_ERR_INVALID, "gelu: null pointer");
	const uint64_t b = (uint64_t)count * 4;
	if (ranges_overlap(y, b, x, b) || ranges_overlap(tanh_saved, b, x, b) || ranges_overlap(tanh_saved, b, y, b))
		return fail(NNH_ERR_ALIAS, "gelu: outputs overlap each other or the input");
	return hip_status(gelu_forward(x, (int64_t)count, y, tanh_saved, reinterpret_cast<hipStream_t>(stream)), "gelu");
}

int nnh_gelu_backward(const float* x, const float* tanh_saved, const float* g, size_t count, float* dx, int first,
                      void* stream) {
	if (!count_ok({count})) return fail(NNH_ERR_INVALID, "gelu backward: size out of range (above 2^60 elements)");
	if (count == 0) return NNH_OK;
	if (!x || !tanh_saved || !g || !dx) return fail(NNH_ERR_INVALID, "gelu backward: null pointer");
	const uint64_t b = (uint64_t)count * 4;
	if (ranges_overlap(dx, b, x, b) || ranges_overlap(dx, b, tanh_saved, b) || partial_overlap(dx, b, g, b))
		return fail(NNH_ERR_ALIAS, "gelu backward: dx overlaps x, the saved tanh or part of g");
	return hip_status(gelu_backward(x, tanh_saved, g, (int64_t)count, dx, first ? 1 : 0,
	                                reinterpret_cast<hipStream_t>(stream)),
	                  "gelu backward");
}

int nnh_embedding_add_forward(const float* weight, size_t V, size_t D, const int* rows, size_t count,
                              const float* addend, size_t addend_rows, float* y, void* stream) {
	uint64_t out = 0;
	if (!count_ok({V, D}) || !count_ok({count, D}, out) || !count_ok({addend_rows, D}))
		return fail(NNH_ERR_INVALID, "embedding add: size out of range (above 2^60 elements)");
	if (out == 0) return NNH_OK;
	if (V == 0) return fail(NNH_ERR_SHAPE, "embedding: empty table");  // every id is out of range (ops.cpp:1999)
	if (addend_rows == 0 || count % addend_rows != 0)
		return fail(NNH_ERR_SHAPE, "embedding add: the addend's rows must divide the ids' count");
	if (!weight || !rows || !y || !addend) return fail(NNH_ERR_INVALID, "embedding add: null pointer");
	if (ranges_overlap(y, out * 4, weight, (uint64_t)V * D * 4) || ranges_overlap(y, out * 4, rows, (uint64_t)count * 4) ||
	    ranges_overlap(y, out * 4, addend, (uint64_t)addend_rows * D * 4))
		return fail(NNH_ERR_ALIAS, "embedding add: y overlaps the table, the rows or the addend");
	return hip_status(embedding_forward(weight, (int64_t)V, (int64_t)D, rows, (int64_t)count, y,
	                                    reinterpret_cast<hipStream_t>(stream), addend, (int64_t)addend_rows),
	                  "embedding add");
}

int nnh_embedding_forward(const float* weight, size_t V, size_t D, const int* rows, size_t count, float* y,
                          void* stream) {
	uint64_t out = 0;
	if (!count_ok({V, D}) || !count_ok({count, D}, out))
		return fail(NNH_ERR_INVALID, "embedding: size out of range (above 2^60 elements)");
	if (out == 0) return NNH_OK;
	if (V == 0) return fail(NNH_ERR_SHAPE, "embedding: empty table");  // every id is out of range (ops.cpp:1999)
	if (!weight || !rows || !y) return fail(NNH_ERR_INVALID, "embedding: null pointer");
	if (ranges_overlap(y, out * 4, weight, (uint64_t)V * D * 4) || ranges_overlap(y, out * 4, rows, (uint64_t)count * 4))
		return fail(NNH_ERR_ALIAS, "embedding: y overlaps the table or the rows");
	return hip_status(embedding_forward(weight, (int64_t)V, (int64_t)D, rows, (int64_t)count, y,
	                                    reinterpret_cast<hipStream_t>(stream)),
	                  "embedding");
}

int nnh_embedding_backward(const float* g, const int* rows, size_t count, size_t V, size_t D, float* dweight, int first,
                           void* stream) {
	uint64_t tab = 0;
	if (!count_ok({V, D}, tab) || !count_ok({count, D}))
		return fail(NNH_ERR_INVALID, "embedding backward: size out of range (above 2^60 elements)");
	if (tab == 0) return NNH_OK;
	if ((uint64_t)V * ((D + 63) / 64) / 4 >= ((uint64_t)1 << 31))  // a wave per row and 64 columns, four to a block
		return fail(NNH_ERR_INVALID, "embedding backward: too many table rows for the grid");
	if (!dweight || (count > 0 && D > 0 && (!g || !rows))) return fail(NNH_ERR_INVALID, "embedding backward: null pointer");
	if (ranges_overlap(dweight, tab * 4, g, (uint64_t)count * D * 4) ||
	    ranges_overlap(dweight, tab * 4, rows, (uint64_t)count * 4))
		return fail(NNH_ERR_ALIAS, "embedding backward: the gradient table overlaps g or the rows");
	return hip_status(embedding_backward(g, rows, (int64_t)count, (int64_t)V, (int64_t)D, dweight, first ? 1 : 0,
	                                     reinterpret_cast<hipStream_t>(stream)),
	                  "embedding backward");
}

}  // extern "C"
