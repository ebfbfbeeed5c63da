// The decoder's projection launches for offset nibbles (Q4b32).
#include "proj_launch.h"

namespace fg {

int launch_proj_q4(const ProjParams &p, int in, int out, bool exact, int nb, size_t smem, unsigned grid, hipStream_t s)
{
    return launch_proj_format<4>(p, in, out, exact, nb, smem, grid, s);
}

}  // namespace fg
