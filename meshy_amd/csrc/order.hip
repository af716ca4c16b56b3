// Document order of a micro-batch's tokens, for doc_ids that are not
// non-decreasing.
//
// The reference's losses sum per document with index_add_ over doc_ids
// (trainer.py:705-848, opd.py:161-197, critic/gae.py:296-312), which accepts
// any order.  The kernels here take each document as one contiguous run of
// tokens (its segment offsets), as both batch layouts produce.  For any
// other order, meshy_doc_order gives the stable sort of the token positions
// by document: perm[k] is the position of the k-th token in document order
// (ties in their original order), sorted_ids[k] its document.  The callers
// gather their per-token inputs through perm, run the kernels on the
// document-ordered copy, and scatter per-token outputs back; the order is a
// function of doc_ids alone, so results stay bitwise reproducible.
//
// The sort is hipCUB's radix sort (stable, LSD) over the key bits that
// n_slots needs, with the positions as values.
#include <hip/hip_runtime.h>

#include <hipcub/hipcub.hpp>

#include "common.h"

namespace meshy {
namespace {

constexpr int kIotaThreads = 256;

__global__ __launch_bounds__(kIotaThreads) void k_iota(int64_t* __restrict__ p, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kIotaThreads + threadIdx.x;
    if (i < n) p[i] = i;
}

// Key bits of ids in [0, n_slots).
int key_bits(int64_t n_slots) {
    int b = 1;
    while (b < 63 && (int64_t{1} << b) < n_slots) ++b;
    return b;
}

// The radix sort's temporary storage (the query runs on the current device).
size_t sort_bytes(int64_t n, int64_t n_slots) {
    size_t bytes = 0;
    if (hipcub::DeviceRadixSort::SortPairs(nullptr, bytes, static_cast<const uint64_t*>(nullptr),
                                           static_cast<uint64_t*>(nullptr), static_cast<const int64_t*>(nullptr),
                                           static_cast<int64_t*>(nullptr), static_cast<int>(n), 0,
                                           key_bits(n_slots), static_cast<hipStream_t>(nullptr)) != hipSuccess)
        return 0;
    return bytes;
}

}  // namespace
}  // namespace meshy

extern "C" size_t meshy_doc_order_workspace_size(int64_t n, int64_t n_slots) {
    using namespace meshy;
    if (n <= 0 || n_slots <= 0 || n > INT32_MAX) return 0;
    const size_t tmp = sort_bytes(n, n_slots);
    if (!tmp) return 0;
    return align_up(sizeof(int64_t) * static_cast<size_t>(n), 256) + align_up(tmp, 256);
}

extern "C" int meshy_doc_order(const int64_t* doc_ids, int64_t n, int64_t n_slots, int64_t* sorted_ids, int64_t* perm,
                               void* workspace, size_t workspace_bytes, hipStream_t stream) {
    using namespace meshy;
    clear_error();
    if (n < 0 || n_slots <= 0) return set_error(MESHY_EINVAL, "meshy_doc_order: bad sizes");
    if (n == 0) return MESHY_OK;
    if (n > INT32_MAX) return set_error(MESHY_EINVAL, "meshy_doc_order: too many tokens");
    if (!doc_ids || !sorted_ids || !perm || !workspace)
        return set_error(MESHY_ENULL, "meshy_doc_order: doc_ids, sorted_ids, perm and workspace are required");
    size_t tmp = sort_bytes(n, n_slots);
    const size_t need = align_up(sizeof(int64_t) * static_cast<size_t>(n), 256) + align_up(tmp, 256);
    if (!tmp || workspace_bytes < need)
        return set_error(MESHY_ESPACE, "meshy_doc_order: workspace needs %zu bytes", need);
    char* p = static_cast<char*>(workspace);
    int64_t* iota = reinterpret_cast<int64_t*>(p);
    void* scratch = p + align_up(sizeof(int64_t) * static_cast<size_t>(n), 256);
    hipLaunchKernelGGL(k_iota, dim3(static_cast<unsigned>(ceil_div(n, kIotaThreads))), dim3(kIotaThreads), 0, stream,
                       iota, n);
    int rc = check_launch("meshy_doc_order(iota)");
    if (rc) return rc;
    // The ids lie in [0, n_slots) (the callers check): as unsigned keys their
    // low key_bits(n_slots) bits order them.
    const hipError_t e = hipcub::DeviceRadixSort::SortPairs(
        scratch, tmp, reinterpret_cast<const uint64_t*>(doc_ids), reinterpret_cast<uint64_t*>(sorted_ids), iota, perm,
        static_cast<int>(n), 0, key_bits(n_slots), stream);
    if (e != hipSuccess) return set_error(static_cast<int>(e), "meshy_doc_order: radix sort failed (%s)",
                                          hipGetErrorString(e));
    return check_launch("meshy_doc_order(sort)");
}
