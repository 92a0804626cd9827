"""ORACLE -- test infrastructure only.

CPU restatement of STAR-KV's paged decode path, the reference results for ``tests/``,
``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py``. The product
(``starkv_serve`` and its HIP library) never imports, links or calls anything here.

* ``quant_oracle.c`` -- the 3.2-bit quantizer and row format, bit for bit (C).
* ``ref.py``         -- row layout, tile tables, block Hadamard, and the decode math
                        in float64 (numpy), plus an emulation of the reference's
                        roundings (torch CPU).

Every function cites the reference file:line it restates. Parity pinning (what
each function is checked against) is listed in ``ref.py``'s header.
"""
