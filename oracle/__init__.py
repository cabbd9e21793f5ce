"""CPU oracle for the decoder-body RMSNorm / RoPE path. TEST INFRASTRUCTURE ONLY: imported by
tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg, never by the product."""
