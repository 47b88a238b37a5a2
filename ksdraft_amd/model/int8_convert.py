"""Model-wide INT8 conversion (mirror of reference ksdraft/model/int8_convert.py:31-52).

``to_int8(model)`` returns a converted copy: Rosa q/k/v/out and ``teacher_proj`` become
``Int8Linear``, each block's KS3 becomes ``KS3Int8Cell``; LayerNorms, the Rosa payload and
time-mix vectors, the DSpine injection and the embedding stay float (the reference's
conversion doctrine). The reference builds the cells without trainable masters
(int8_convert.py:40); ``trainable=True`` builds them with masters and also turns the tied
head into an ``Int8Linear`` sharing the embedding's weight, so every linear of the step
runs INT8 forward and backward (the config-5 training step). ``int8_embedding=True``
also swaps the embedding lookup for the int8 gather over the head's codes, and
``int8_injection=True`` the DSpine injection's low-rank maps for Int8Linear (their rank-32/64
reductions pad to one 128-wide group, quant.py:9-10): the staged surfaces the reference's
doctrine keeps float until gated.
"""

from __future__ import annotations

import copy

from ..kernels.embedding import Int8Embedding
from ..kernels.ks3_int8 import KS3Int8Cell
from ..kernels.linear import Int8Linear
from .draft import KSDraftModel


def to_int8(model: KSDraftModel, group: int = 128, nonlinear: str = "int8", *,
            trainable: bool = False, int8_embedding: bool = False,
            int8_injection: bool = False) -> KSDraftModel:
    conv = copy.deepcopy(model)
    swapped = 0
    for block in conv.blocks:
        rosa = block.rosa
        for name in ("q_proj", "k_proj", "v_proj", "out_proj"):
            setattr(rosa, name, Int8Linear.from_float(getattr(rosa, name)))
            swapped += 1
        block.ffn = KS3Int8Cell(cell=block.ffn, group=group, nonlinear=nonlinear,
                                trainable=trainable)
        swapped += 1
        if int8_injection:  # DSpine's low-rank maps: reduction 32/64 pads to one group
            inj = block.injection
            for name in ("feature_down", "feature_up"):
                setattr(inj, name, Int8Linear.from_float(getattr(inj, name)))
                swapped += 1
            for lr in (inj.gate_q, inj.gate_p, inj.inject):
                lr.down = Int8Linear.from_float(lr.down)
                lr.up = Int8Linear.from_float(lr.up)
                swapped += 2
    if conv.teacher_proj is not None:
        conv.teacher_proj = Int8Linear.from_float(conv.teacher_proj)
        swapped += 1
    if trainable:
        head = Int8Linear(conv.head.in_features, conv.head.out_features, bias=False)
        head.weight = conv.embedding.weight   # tied, as KSDraftModel ties its head
        head.weight_codes = head.weight_scales = None
        conv.head = head
        swapped += 1
    if int8_embedding:  # the staged int8-embedding surface: lookups from the head's codes
        emb = Int8Embedding.from_float(conv.embedding, group)
        if isinstance(conv.head, Int8Linear):
            emb.codes_from = conv.head
        conv.embedding = emb
        swapped += 1
    conv._int8_tier = {"group": group, "nonlinear": nonlinear, "swapped_surfaces": swapped,
                       "trainable": trainable, "int8_embedding": int8_embedding,
                       "int8_injection": int8_injection}
    return conv


def int8_surfaces(converted: KSDraftModel) -> dict:
    info = getattr(converted, "_int8_tier", None)
    return dict(info) if info else {}
