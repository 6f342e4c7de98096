"""CPU oracle for the paged-KV attention path.

TEST INFRASTRUCTURE ONLY: the checker.  Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg may import it; the product library
(qauntrunner_amd, libqr_attn.so) never does.
"""
