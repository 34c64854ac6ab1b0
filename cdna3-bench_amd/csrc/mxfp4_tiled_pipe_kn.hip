// The pipelined tiled kernel's KN instantiations (one translation unit
// per weight layout: see mxfp4_tiled_pipe.h).
#include "mxfp4_tiled_pipe.h"

namespace mxfp4 {

hipError_t launch_tiled_pipe_kn(const TiledShape& shape, const TiledArgs& args, hipStream_t stream) {
  return dispatch_shape<kLayoutKN>(shape, args, stream);
}

}  // namespace mxfp4
