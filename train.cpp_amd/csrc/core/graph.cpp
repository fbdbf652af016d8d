// Graph construction: iterative post-order walk over the sources, so every
// node appears after all of its inputs (the reference's order,
// src/core/trc_graph.cpp:40-77).
#include "impl.h"

namespace traincpp {

Graph* graph_new(Context* ctx) {
    TRC_CHECK(ctx != nullptr, "graph_new: ctx is NULL");
    Graph* g = new Graph();
    g->ctx = ctx;
    return g;
}

void graph_free(Graph* graph) {
    delete graph;
}

void graph_clear(Graph* graph) {
    graph->nodes.clear();
    graph->leafs.clear();
    graph->visited.clear();
    graph->backward_built = false;
}

void graph_build_forward_expand(Context* ctx, Graph* graph, Tensor* tensor) {
    TRC_CHECK(ctx == graph->ctx, "graph_build_forward_expand: tensor context differs from the graph's");
    if (tensor == nullptr) return;
    // (tensor, index of the next source to visit)
    std::vector<std::pair<Tensor*, int>> stack{{tensor, 0}};
    while (!stack.empty()) {
        auto& [node, next] = stack.back();
        // a node's sources end at its first null entry (src/core/trc_graph.cpp:59-61)
        if (next < node->nsrc && node->src[next] != nullptr) {
            Tensor* s = node->src[next++];
            if (!graph->visited.count(s)) stack.push_back({s, 0});
            continue;
        }
        Tensor* done = node;
        stack.pop_back();
        if (graph->visited.insert(done).second) {
            graph->nodes.push_back(done);
            if (done->nsrc == 0) graph->leafs.push_back(done);
        }
    }
}

int64_t graph_n_nodes(const Graph* graph) {
    return (int64_t) graph->nodes.size();
}

Tensor* graph_node(const Graph* graph, int64_t index) {
    TRC_CHECK(index >= 0 && index < (int64_t) graph->nodes.size(), "graph_node: index out of range");
    return graph->nodes[(size_t) index];
}

int64_t graph_n_leafs(const Graph* graph) {
    return (int64_t) graph->leafs.size();
}

Tensor* graph_leaf(const Graph* graph, int64_t index) {
    TRC_CHECK(index >= 0 && index < (int64_t) graph->leafs.size(), "graph_leaf: index out of range");
    return graph->leafs[(size_t) index];
}

}  // namespace traincpp
