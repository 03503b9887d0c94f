"""CPU oracle of the Allie policy/value inference path -- TEST INFRASTRUCTURE.

This package is a checker.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import it; the product
(``allie_amd``) never does, and it is never the thing measured on the GPU.

Contents and what pins each part (details in each module's docstring):

* ``pack_ref.c`` / ``pack.py`` -- ragged packing (data.py:281-337 restated
  for a flat token stream).  Pinned against the padded ``pad_and_collate``
  formulas (cumsum positions, ``& 0x3FFF`` ids) and closed-form invariants.
* ``model_ref.py`` -- the model forward (model.py:13-147 plus the GPT-2
  [lib] block arithmetic) in fp32 torch on the CPU, and a bf16-autocast
  emulation.  Pinned by a float64 numpy brute force at tiny shapes, by
  transformers' own GPT2LMHeadModel built from a local config with the same
  weights (fp32, and under torch.autocast for the bf16 mode), and by closed
  forms for the Elo control embedding.
* ``movegen.py`` -- the rules of chess in Python (python-chess's behaviour
  behind data.py:51-61 and decode.py:345-353), the comparator of the native
  rules library; legality pinned by perft known answers, move order
  unpinned (python-chess is absent).

The decode strategies' scalar maths (decode.py:381-467, 503-516) are checked
in tests/test_decode.py against closed forms and a float64 bisection.
"""
