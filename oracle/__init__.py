"""CPU oracle for the quantized linear-layer path. Test infrastructure only:
imported by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg,
never by the hydraserve_amd package."""
