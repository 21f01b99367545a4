"""Host-side launchers of the MoBA pipeline, in the order the forward runs:

    pooling   mean-pool each key block into one representative key
    gating    score queries against the representatives, keep top-k
    routing   transpose the choice into per-block columns (CSC)
    moba_fwd  attend per (KV block, kv head), then merge per-slot partials
    moba_bwd  the backward of the same
    attention the two halves as one differentiable operation

Every launcher calls the HIP library (`moba._lib`); none has a CPU path.
"""
