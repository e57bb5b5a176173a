"""CPU oracle of the block-sparse causal attention forward — TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, to check
results or as the timed CPU port; never by the usagi_amd package.

  bsa_oracle.dense_masked   numpy fp32/fp64 dense-masked softmax attention (math oracle)
  bsa_oracle.blockwise_v7   numpy restatement of the reference CSR walk
  c_ref.fwd                 plain-C restatement of the same walk (oracle/bsa_ref.c), OpenMP
"""
