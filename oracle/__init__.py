"""CPU oracle of the strands-decider torso: TEST INFRASTRUCTURE ONLY.

oracle.c restates the reference's WGSL kernels (mircodz/strands-decider-rs, src/kernels.rs) in C;
torso.py composes them the way the reference's plan does (src/engine.rs:396-662).  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and only as the
checker or the timed CPU baseline; the product (strands-decider-rs_amd, libsdhip.so) never does.
"""
