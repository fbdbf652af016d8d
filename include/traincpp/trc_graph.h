// traincpp-compatible computation graph. Interface of include/traincpp/trc_graph.h
// in the reference: nodes in post-order (every source before its consumer).
#pragma once

#include "trc_tensor.h"

#include <unordered_set>
#include <vector>

namespace traincpp {

struct Graph {
    Context* ctx = nullptr;
    std::vector<Tensor*> nodes;   // post-order
    std::vector<Tensor*> leafs;   // nodes without sources
    std::unordered_set<Tensor*> visited;
    bool backward_built = false;
};

Graph* graph_new(Context* ctx);
void   graph_free(Graph* graph);
void   graph_clear(Graph* graph);
void   graph_build_forward_expand(Context* ctx, Graph* graph, Tensor* tensor);

int64_t graph_n_nodes(const Graph* graph);
Tensor* graph_node(const Graph* graph, int64_t index);
int64_t graph_n_leafs(const Graph* graph);
Tensor* graph_leaf(const Graph* graph, int64_t index);

}  // namespace traincpp
