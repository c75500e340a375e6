"""CPU checker for the HIP engine. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only to check or to time the CPU path; the engine
(bnns_to_c_amd) never imports it.
"""
