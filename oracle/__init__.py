"""CPU oracle for the W4A8 matvec path -- TEST INFRASTRUCTURE ONLY.

Nothing in the product package (`fable5_llm_amd`) imports this package.  Only
`tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py`
may use it, and only to check results against or as the timed CPU
baseline, never as a fallback for the HIP path.

Contents
  law.py     numpy restatement of the reference's integer law (each function
             cites the reference file:line it follows)
  law_c.c    plain-C restatement of the hot loops (matvec over a wire image,
             DYNQ8, argmax) -- an independent second implementation and the
             multi-threaded CPU baseline; built by oracle/Makefile into
             oracle/liboracle_w4a8.so
  cfast.py   ctypes loader for law_c.c
  fixtures.py loaders for the committed golden vectors under tests/golden/

Parity status of every function is recorded in law.py's module docstring.
"""
