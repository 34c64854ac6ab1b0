// Entry points of the pipelined tiled kernel (mxfp4_tiled_pipe.h); the
// per-layout instantiations live in mxfp4_tiled_pipe_{kn,nk,g,p}.hip.
#include "mxfp4_kernels.h"
#include "mxfp4_tiled_pipe.h"

namespace mxfp4 {

hipError_t launch_tiled_pipe_kn(const TiledShape& shape, const TiledArgs& args, hipStream_t stream);
hipError_t launch_tiled_pipe_nk(const TiledShape& shape, const TiledArgs& args, hipStream_t stream);
hipError_t launch_tiled_pipe_g(const TiledShape& shape, const TiledArgs& args, hipStream_t stream);
hipError_t launch_tiled_pipe_p(const TiledShape& shape, const TiledArgs& args, hipStream_t stream);

bool tiled_pipe_shape_available(int layout, const TiledShape& s) {
  (void)layout;
#define X(WM_, WN_, RB_, WNC_, NS_) \
  if (s.wm == WM_ && s.wn == WN_ && s.rb == RB_ && s.wnc == WNC_ && s.stages == NS_) return true;
  MXFP4_PIPE_SHAPES(X)
#undef X
  return false;
}

hipError_t launch_tiled_pipe(int layout, const TiledShape& shape, const TiledArgs& args,
                             hipStream_t stream) {
  switch (layout) {
    case kLayoutKN: return launch_tiled_pipe_kn(shape, args, stream);
    case kLayoutNK: return launch_tiled_pipe_nk(shape, args, stream);
    case kLayoutG: return launch_tiled_pipe_g(shape, args, stream);
    case kLayoutP: return launch_tiled_pipe_p(shape, args, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mxfp4
