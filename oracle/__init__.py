"""CPU oracle for the streaming semi-Markov scan -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference computes on the hot path
(biobenkj/torch-semimarkov, ``src/torch_semimarkov/streaming/pytorch_reference.py``,
``streaming/autograd.py`` and ``nn.py``).  It is the *checker* for the HIP
kernels: only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may import it.  The product package
(``torch_semimarkov_amd``) never imports it and never falls back to it.

Modules
-------
streaming_ref
    dtype-generic PyTorch-CPU restatement of the reference forward (log/max),
    checkpointed backward, Viterbi traceback and gold-path scoring.  In fp32 it
    reproduces the reference's arithmetic order (the per-step ``logsumexp``
    inputs are the same tensors the reference stacks); in fp64 it is the
    accuracy yardstick for long sequences.
brute
    Independent checks that pin ``streaming_ref``: exhaustive enumeration of
    all segmentations for tiny problems (log Z, Viterbi, exact marginals via
    autograd) and a textbook HMM forward/backward for the K=1 special case.

Pinning status of each function is recorded in each module's docstring.
"""
