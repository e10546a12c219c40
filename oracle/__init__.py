"""ORACLE -- test infrastructure only.

CPU restatements of the reference's routed-expert MoE layer, used as the checker by
``tests/``, by ``__graft_entry__.smoke()`` and by the CPU-baseline leg of ``bench.py``.
Nothing in the ``kandiga_amd`` package imports, links or calls this package; the
product path runs only the HIP library and fails if it is missing.

Pins (each function's docstring names its checks in ``tests/``):

* ``unpack_codes``      known-answer byte patterns, pack/unpack round trip, the BKEX
                        offset constants of kandiga_cpu_expert.m:42-65.
* ``dequantize``        closed form ``(q - 2**(b-1)) * s`` exact for the synthetic scales;
                        element-by-element brute force (codes read bit by bit) on general,
                        independent fp16/bf16 scale/bias pairs.
* ``route``             brute force over E on small inputs, softmax identities, tie cases,
                        NaN and infinite logits.
* ``permute``           brute-force ``sorted(range(T*K), key=(expert, flat index))``.
* ``combine``           closed form ``sum_k w_k y_k``, linearity.
* ``switch_mlp`` (C)    float64 numpy matmul over fully dequantized matrices
                        (``expert_mlp_f64``), zero-weight and one-hot special cases; the
                        GELU-tanh mode against ``torch.nn.functional.gelu(approximate='tanh')``.
* ``shared_expert_f64`` closed form for constant matrices (with a gate/up swap that must
                        differ) and explicit index loops on non-square matrices.
* ``qlinear_f64``       brute-force loops over the quantized rows.
* ``moe_block``         the block composition against a closed form with constant shared
                        weights.
* ``ref_scalar`` (C)    the same layer as ``switch_mlp`` within fp32 rounding.
* ``tq3_oracle``        Hadamard identities (H H = 32 I, inverse of forward, the dot identity),
                        the sign table's defining hash, centroid/boundary consistency, a
                        constant block's closed form, index packing, and the reference
                        quantizer's own blocks and dequantized weights
                        (tests/golden/tq3_quantize.npz).
"""
