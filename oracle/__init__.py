"""CPU oracle for the quantized decode GEMV path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package.  It is the checker for the HIP kernels, never part of the product path.
"""
