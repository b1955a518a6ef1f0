"""CPU oracle for the Mamba-1 op set — TEST INFRASTRUCTURE ONLY.

Nothing in the product (`mamba-cpu_amd/`) imports, links or runs anything here.
Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` use it, and only as the checker / the timed CPU reference.

Contents
  oracle.numerics  float64 numpy restatement of the reference's algorithms
                   (forward and analytic backward of the selective scan,
                   causal conv1d forward/backward/update, state update).
  oracle.ref       ctypes loader for oracle/_ref/libmcpu_ref.so, the
                   reference's own C++ CPU kernels compiled from the reference
                   sources by oracle/Makefile.
  oracle.cpu_torch the reference's CPU execution path for timing (its ATen
                   conv / state-update code paths, an autograd wrapper around
                   oracle.ref's kernels, and its transformers routing).

Pinning (how each oracle function is checked, so a plausible mistake fails):
  scan forward      vs the compiled reference (_ref) on random inputs; closed
                    forms (delta=0 -> out = D*u; A=-inf -> memoryless state;
                    dstate=1 hand recurrence); NaN confinement.
  scan backward     vs the compiled reference (_ref); vs torch.autograd through
                    an independent float64 forward; central finite differences.
  complex-A scan    (mamba_ssm's semantics; the reference has no complex path)
                    forward vs a closed-form direct sum and vs the real scan
                    (Im A = 0); a phase invariance of B/C; backward vs
                    torch.autograd through the direct sum in complex128.
  conv forward      vs numpy.convolve per channel (textbook routine);
                    initial/final-state chaining invariants.
  conv backward     vs torch.autograd through F.conv1d in float64.
  conv update       update steps == full conv (invariant); state == last inputs.
  state update      L single steps == full scan (whose oracle is pinned above);
                    multi-head layout == flattened layout.
  cpu_torch         each function vs the pinned float64 functions above
                    (tests/test_cpu_baseline.py).
Every function is pinned; none is "parity unpinned".
"""
