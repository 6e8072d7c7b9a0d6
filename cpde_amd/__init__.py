"""MI355X-native cPDE: gfx950 kernels for the derivative-stack training epoch
behind a C ABI (include/cpde_hip.h), a protocol server speaking the cPDE wire
format, and Python bindings used by the tests and the benchmark."""
