"""CPU oracle for the FADE tiered-KV hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the arithmetic of the reference FADE
implementation (Omodaka9375/fade, pure Python over torch) for the three
hot-path pieces: INT4/INT2 quantize + bit-pack, the eviction re-RoPE rewrite
of surviving keys, and attention over a dequantized tiered cache.  Each
function cites the reference file:line it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker (or the
timed CPU baseline).  The product (``fade_amd``) never imports it: its
kernels run on the GPU through ``libfade_hip.so`` and fail loudly without it.

Rounding model.  The reference evaluates fp16 tensors with torch CPU ops,
which compute each op in fp32 and round the result to fp16 (probed for
every positive finite fp16 input, see ``tests/test_oracle_pins.py``).  The
oracle reproduces that with explicit ``astype(np.float32)`` /
``astype(np.float16)`` pairs around every op.

Pinning status (what checks each function; details in the tests):
  pack/unpack INT4, INT2      brute force over every nibble pair / 2-bit quad
  quant_*_int4, quant_*_int2  exhaustive torch-op rounding probes + invariants
  rotated quant               invariants; quantizer exact given x_rot
  asym group quant            build-defined format (no reference counterpart):
                              invariants only -- parity with the reference
                              is unpinned because the reference has no such
                              format
  rope tables / re-RoPE       closed forms (inverse(apply) ~ identity,
                              identity at unchanged positions) + torch probe
  assign_one_layer            the reference's own known-answer test + brute
                              force
  attention                   textbook softmax attention, brute force on
                              tiny shapes, uniform-key closed form
"""
