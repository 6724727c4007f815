// Work partition of the one-launch decode layer kernel (stream_fp8.hip),
// shared by the kernel and a host-side test (compiled with a plain C++
// compiler: no HIP-only code here).
//
// Each phase splits its items -- n_act active experts x ipe items per
// expert, expert-major -- into nwg contiguous ranges of ceil(total / nwg)
// items; workgroup b runs gate_up range b, then down range b.  A down range
// waits for every gate_up range holding an item of one of its experts:
// layer_dependencies gives them as the interval [*lo, *hi] (empty: hi < lo).
#pragma once

#if defined(__HIPCC__)
#define MSTAR_HD __host__ __device__
#else
#define MSTAR_HD
#endif

namespace mstar {

// Items [*i0, *i1) of range r.
MSTAR_HD inline void layer_range(int n_act, int ipe, int nwg, int r, int* i0, int* i1) {
  const int total = n_act * ipe;
  const int t = (total + nwg - 1) / nwg;
  *i0 = r * t;
  *i1 = *i0 + t < total ? *i0 + t : total;
  if (*i1 < *i0) *i1 = *i0;
}

// Gate_up ranges (ipe1 items per expert) down range r (ipe2 per expert) waits on.
MSTAR_HD inline void layer_dependencies(int n_act, int ipe1, int ipe2, int nwg, int r, int* lo, int* hi) {
  *lo = 0;
  *hi = -1;
  int d0, d1;
  layer_range(n_act, ipe2, nwg, r, &d0, &d1);
  const int t1 = (n_act * ipe1 + nwg - 1) / nwg;
  if (d0 >= d1 || t1 <= 0) return;
  *lo = (d0 / ipe2) * ipe1 / t1;
  const int h = (((d1 - 1) / ipe2 + 1) * ipe1 - 1) / t1;
  *hi = h < nwg - 1 ? h : nwg - 1;
}

}  // namespace mstar
