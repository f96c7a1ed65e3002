// ggml_impl.h - libgcq-internal definitions shared by the ggml API's graph construction (ggml.hip)
// and its HIP backend (ggml_backend.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <string>
#include <unordered_set>
#include <vector>

#include "../../include/ggml-alloc.h"
#include "../../include/ggml-backend.h"
#include "../../include/ggml.h"

struct ggml_context {
    bool no_alloc = true;
    std::vector<ggml_tensor *> tensors;  // owned, in creation order
    std::vector<void *> host_data;       // owned host memory of no_alloc == false tensors
    std::vector<ggml_cgraph *> graphs;   // owned
};

struct ggml_cgraph {
    size_t size = GGML_DEFAULT_GRAPH_SIZE;
    std::vector<ggml_tensor *> nodes;  // in execution order
    std::vector<ggml_tensor *> leafs;
    std::unordered_set<const ggml_tensor *> visited;
    std::string error;  // a NULL tensor was expanded: the reason it is NULL
};

namespace gcq {

// Element counts of a type's block and bytes of one block (0 for a type this library does not
// know). Shared with the C ABI's size functions.
int64_t ggml_blck(int type);
size_t ggml_tsize(int type);

// The tensor owning t's memory (t itself if it is not a view).
inline const ggml_tensor * base_of(const ggml_tensor * t) { return t->view_src ? t->view_src : t; }
inline bool is_view_op(int op) {
    return op == GGML_OP_VIEW || op == GGML_OP_RESHAPE || op == GGML_OP_PERMUTE || op == GGML_OP_TRANSPOSE;
}
// A Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K tensor in this library's device buffers: stored packed (gcq_pack_weights).
inline bool is_packed_type(int t) {
    return t == GGML_TYPE_Q4_0 || t == GGML_TYPE_Q8_0 || t == GGML_TYPE_Q4_K || t == GGML_TYPE_Q5_K || t == GGML_TYPE_Q6_K;
}

// Fusion chains of a graph (ggml_backend.hip): end[i] is the node index at which node i's work
// runs (i itself, or the last node of the chain it starts or belongs to; for a folded norm, its
// last reader); member[i] is true for a node whose result is folded into later nodes and never
// materialized.
struct Chains {
    std::vector<int> end;
    std::vector<bool> member;
    // mul(rms_norm(x), w) rows of one row folded into each of their GEMV readers (x and w are
    // read by every reader; the norm and the mul are members).
    std::vector<const ggml_tensor *> folded;
    std::vector<bool> in_fold;  // the norm and mul nodes of a folded row
    // GEMVs of one folded row with no residual add (q / k / v, gate / up): run as one launch at
    // the first one's place, their results all placed there (sib[i]: group of node i, or -1).
    std::vector<std::vector<int>> groups;
    std::vector<int> sib;
    // group kinds: 0 the GEMVs above; 1 two ropes (q, k) and 2 two set_rows (k, v) of the same
    // positions, the second's input computed before the first: one launch at the first's place.
    std::vector<int> kind;
    // kind 3: q / k / v GEMVs of one row with the decode step's rope of q and k and the set_rows of
    // k and v into f16 caches, as one launch: {mm_q, mm_k, mm_v, rope_q, then the reshape / rope /
    // permute / set_rows members}; only rope_q's result is written to memory of its own.
    // kind 4: gate / up GEMVs of one row read only by a swiglu, as one launch writing the swiglu's
    // result: {mm_gate, mm_up, glu}; only the glu's result has memory of its own.
    std::vector<int> first;  // each group's earliest node: where its launch runs
};
Chains find_chains(const ggml_cgraph * g, bool fuse = true);

// The HIP backend's stream for work a driver orders around its graphs, and graph computes that
// do not wait for the graph (ggml_backend_graph_compute does). backend_set_fusion(false): every
// node planned alone and given memory of its own (node-by-node profiling).
enum ggml_status graph_compute_async(ggml_backend_t backend, ggml_cgraph * cgraph);
hipStream_t backend_stream(ggml_backend_t backend);
// Changes whenever the executor's workspace moves: graphs captured over its launches before then
// read the old workspace.
uint64_t backend_epoch(ggml_backend_t backend);
void backend_activate(ggml_backend_t backend);
void backend_set_fusion(ggml_backend_t backend, bool on);

}  // namespace gcq
