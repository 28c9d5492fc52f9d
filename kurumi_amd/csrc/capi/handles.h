// Opaque C-ABI handle layouts (kurumi/src/capi.rs:27-33 analog), shared by the library and
// by out-of-library consumers that operate on the same graph/tensor handles.
#pragma once

#include <memory>
#include "../ir/graph.h"
#include "../ir/tensor.h"

struct KuGraph { ku::Graph g; };
// Immutable once made (no C entry point writes into a tensor), so a feed shares it instead of
// copying its bytes.
struct KuTensor { std::shared_ptr<const ku::Tensor> t; };
inline KuTensor* new_ku_tensor(ku::Tensor&& x) { return new KuTensor{std::make_shared<const ku::Tensor>(std::move(x))}; }
struct KuFeeds { ku::Feeds f; };
