// The geometry of one forward pass (src/plan.rs:31-113 of the reference).
//
// The GPU path keeps no host index maps: the window partition with its cyclic
// roll, the OCAB unfold and the shift mask are computed in the kernels' load
// and store addressing. What remains on the host is the plan itself and the
// closed-form relative-position indices written into generated checkpoints.
#pragma once
#include <cstdint>
#include <vector>

namespace hat {

struct Plan {
    int h = 0, w = 0;    // input size
    int hp = 0, wp = 0;  // padded to a window multiple
    int c = 0, win = 0, shift = 0, owin = 0;

    static Plan make(int h, int w, int win, int c)
    {
        Plan p;
        p.h = h;
        p.w = w;
        p.hp = (h + win - 1) / win * win;
        p.wp = (w + win - 1) / win * win;
        p.c = c;
        p.win = win;
        p.shift = win / 2;
        p.owin = win + win / 2;
        return p;
    }
    long tokens() const { return (long)hp * wp; }
    int nx() const { return wp / win; }
    int ny() const { return hp / win; }
    int nw() const { return nx() * ny(); }
    int opad() const { return (owin - win) / 2; }
    bool operator==(const Plan& o) const
    {
        return h == o.h && w == o.w && hp == o.hp && wp == o.wp && c == o.c && win == o.win;
    }
};

// relative_position_index_SA as the reference registers it
// (hat_arch.py:882-895): (query - key) + (win - 1) per axis.
inline std::vector<int64_t> rpi_sa_raw(int win)
{
    const int n = win * win;
    std::vector<int64_t> out((size_t)n * n);
    for (int qy = 0; qy < win; ++qy)
        for (int qx = 0; qx < win; ++qx)
            for (int ky = 0; ky < win; ++ky)
                for (int kx = 0; kx < win; ++kx)
                    out[(size_t)(qy * win + qx) * n + ky * win + kx] =
                        (int64_t)(qy - ky + win - 1) * (2 * win - 1) + (qx - kx + win - 1);
    return out;
}

// relative_position_index_OCA (hat_arch.py:897-919): (key - query) +
// (win - owin + 1) per axis, NOT folded: the raw buffer holds negatives that
// PyTorch's indexing wraps from the end of the table.
inline std::vector<int64_t> rpi_oca_raw(int win, int owin)
{
    const int nk = owin * owin, side = win + owin - 1, sh = win - owin + 1;
    std::vector<int64_t> out((size_t)win * win * nk);
    for (int qy = 0; qy < win; ++qy)
        for (int qx = 0; qx < win; ++qx)
            for (int ky = 0; ky < owin; ++ky)
                for (int kx = 0; kx < owin; ++kx)
                    out[(size_t)(qy * win + qx) * nk + ky * owin + kx] =
                        (int64_t)(ky - qy + sh) * side + (kx - qx + sh);
    return out;
}

}  // namespace hat
