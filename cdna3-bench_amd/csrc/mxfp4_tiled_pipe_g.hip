// The pipelined tiled kernel's G instantiations (one translation unit
// per weight layout: see mxfp4_tiled_pipe.h).
#include "mxfp4_tiled_pipe.h"

namespace mxfp4 {

hipError_t launch_tiled_pipe_g(const TiledShape& shape, const TiledArgs& args, hipStream_t stream) {
  return dispatch_shape<kLayoutG>(shape, args, stream);
}

}  // namespace mxfp4
