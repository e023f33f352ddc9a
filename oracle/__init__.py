"""CPU oracle for the Spider-MoE block — TEST INFRASTRUCTURE ONLY.

This package restates the reference's Spider-MoE block on the CPU so that the
HIP path can be checked against it.  Only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s CPU-baseline leg may import it, and only as the checker or
as the timed CPU baseline: the product (``spider-web-moe_amd/``) never imports,
links or calls anything here.

Modules
-------
quant   int4 / fp8-e4m3 weight formats (numpy, integer / byte arithmetic)
plan    dispatch plan: per-expert token lists (numpy, integer)
block   router, edge generator, message pass, expert FFN, epilogue, block
        forward (torch on the CPU, float32 math)
lm      the SpiderWebLM shell around the block (attention prelude / coda)
ref     ctypes binding of the reference's own scalar C++ library, compiled
        from its sources into ``oracle/_ref`` by ``oracle/Makefile``

Parity pins (what checks each oracle function against something other than
itself) are listed in each module's docstring.  Functions without such a
check say "parity unpinned".
"""
