// Exports the reference's own poly7 sin family, compiled from its header
// where it lies (compiler/include/mlk/support/math_families.h), so the
// oracle's restatement can be checked bit-for-bit against it. Test
// infrastructure only: built into oracle/_ref/ when /root/reference exists.
#include "mlk/support/math_families.h"

extern "C" double ref_poly_sin(double x) { return mlk::families::polySin(x); }

extern "C" double ref_measured_poly_sin_max_ulps() {
    return mlk::families::measuredPolySinMaxUlps();
}
