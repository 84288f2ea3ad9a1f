"""CPU oracle of the weight-streaming path.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` import this package, and only as the
checker. The product package (``flextensor_amd``) never imports it.

Each module restates one part of the reference (ai-dynamo/flextensor 0.5.0,
a pure-Python library) and cites the file:line it follows:

* ``layout``       packed byte layout, dense-layout test, typed views
* ``planner``      slot colouring and schedule surgery (block planner,
                   strategy operations, block-strategy glue)
* ``schedule``     stream/event operation traces of the transfer runtime and
                   both pipelined loaders, replayed on a recording fake stream
* ``interpolator`` log-log size <-> duration link model
* ``timing``       per-pass totals, per-trap report statistics and the hidden
                   fraction of the offload timing
* ``fp8``          float8 e4m3fn decoding (OCP format definition) and the
                   fp8-weight linear layer in float64
* ``native``       ctypes access to ``liboracle.so`` (plain C: layout, pack,
                   scatter, checksum)
* ``expcode``      the exponent-coded block format of encoded streamed
                   blocks (this build's own format, no reference counterpart)
* ``expcode_dense`` the dense exponent-coded format (v2) of units kept
                   encoded in HBM (this build's own, no reference counterpart)
"""
