// Opaque C-ABI handle layouts (kurumi/src/capi.rs:27-33 analog), shared by the library and
// by out-of-library consumers that operate on the same graph/tensor handles.
#pragma once
#include "../ir/graph.h"
#include "../ir/tensor.h"

struct KuGraph { ku::Graph g; };
struct KuTensor { ku::Tensor t; };
struct KuFeeds { ku::Feeds f; };
