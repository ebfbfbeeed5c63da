// The decoder's projection launches for 8-bit levels (Q7b32, Q8b32).
#include "proj_launch.h"

namespace fg {

int launch_proj_q8(const ProjParams &p, int in, int out, bool exact, int nb, size_t smem, unsigned grid, hipStream_t s)
{
    return launch_proj_format<8>(p, in, out, exact, nb, smem, grid, s);
}

}  // namespace fg
