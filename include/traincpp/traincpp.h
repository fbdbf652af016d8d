// Umbrella header of the traincpp-compatible API subset shipped with the
// MI355X HIP backend.
#pragma once

#include "trc_backend.h"
#include "trc_context.h"
#include "trc_gguf.h"
#include "trc_graph.h"
#include "trc_hip.h"
#include "trc_op.h"
#include "trc_ops.h"
#include "trc_tensor.h"
#include "trc_types.h"
