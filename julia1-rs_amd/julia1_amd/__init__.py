"""Host-side Python mirror of the julia1 encoder-forward interface over the
MI355X (gfx950) HIP backend: ctypes bindings of libjulia1_hip.so (`hip`),
the checkpoint/batch structures (`abi`) and seeded synthetic workloads (`synth`)."""
