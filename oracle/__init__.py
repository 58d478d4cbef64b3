"""CPU oracle for the pico-hip decode path.

TEST INFRASTRUCTURE ONLY. Nothing in the product (the ``pico_hip`` package,
``libpico_hip.so``) imports, links or calls anything here. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use
this package, and only as the checker / the reported CPU baseline, never as the
thing measured or shipped.

Contents (each function cites the reference file:line it restates):

* ``dequant``  -- numpy restatement of the GGML block formats and the
  reference's int8+scale "unpacked" kernel form (``src/pico_engine/dequant.py``).
* ``dequant_ref.c`` -- an independent C restatement of the same block decode,
  built by ``oracle/Makefile`` into ``oracle/_build/liboracle_dequant.so``;
  used to cross-check the numpy restatement bit for bit.
* ``ref_cpu``  -- a torch-CPU restatement of the reference's dense Qwen2
  forward (``src/pico_engine/model.py``, ``kernels.py``), used as the end-to-end
  oracle for greedy tokens and as the timed CPU baseline.
* ``closed``   -- float64 closed forms (GEMV, attention, RMSNorm, RoPE) used to
  pin the kernels and ``ref_cpu``.

Pinning status of every function is listed in the module docstrings; there is
no function marked "parity unpinned" at present.
"""
