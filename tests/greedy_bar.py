"""A greedy-token parity bar derived from the oracle's own disagreement (GPU tests).

The reference samples greedy tokens as torch.argmax over the bf16 logits of its bf16 model
(nv/layers/sampler.py:13-14, nv/models/qwen3.py:203-221): on random-weight models the top two
logits are often one bf16 step apart or equal, so which token wins depends on the summation order
of every product and sum before them.  Two correct evaluations of the same model therefore
disagree on some tokens, and the product may not be held to more than that.

``legal_variants`` evaluates the oracle four legal ways on the product's own token stream
(teacher-forced, so every evaluation sees the same history): fp32 arithmetic (the oracle proper),
fp64 arithmetic, and each of them with the softmax probabilities rounded to bf16 before the PV
product (what a kernel that runs PV on a bf16 matrix unit does).  ``check`` measures, from those runs:

* ``legal_mismatch``: the largest number of tokens two variants choose differently;
* ``legal_step_diff[s]``: the largest logit difference between two variants at step s (any row);
* ``legal_std``: the range of the std of the logit differences between two variants;

and asserts that
1. the product's tokens differ from the fp32 oracle's no more often than the variants differ from
   each other, plus two standard deviations of that count (a Poisson count n: 2 sqrt(n), at least 2);
2. every product token that differs sits at a step where the oracle's margin (its top logit minus
   the product token's) is no larger than two legal evaluations' logits differ at that step;
3. the std of the product's logit difference from the oracle is within the variants' range, widened
   by that range's own width.
A systematic error (a wrong scale, a dropped term) raises the logit difference and the mismatch
count past these bars; rounding-order noise does not.
"""
from __future__ import annotations

import itertools
import math

import torch

from oracle.qwen3_ref import Qwen3Ref


def legal_variants(state, config, prompts, tokens, device, max_positions=512):
    """Teacher-forced bf16-mode oracle logits [rows, steps, vocab] of the four legal evaluations.
    Rows whose prompts have one length advance together through ``forward_batch``."""
    steps = len(tokens[0])
    kinds = {"fp32": dict(), "fp64": dict(dtype=torch.float64), "fp32_bf16_probs": dict(round_probs=True),
             "fp64_bf16_probs": dict(dtype=torch.float64, round_probs=True)}
    groups: dict[int, list[int]] = {}
    for i, p in enumerate(prompts):
        groups.setdefault(len(p), []).append(i)
    out = {}
    for name, kw in kinds.items():
        ref = Qwen3Ref(state, config, round_bf16=True, max_positions=max_positions, device=device, **kw)
        rows = [None] * len(prompts)
        for idx in groups.values():
            ref.reset(len(idx))
            logits = [ref.forward_batch([list(prompts[i]) for i in idx]).cpu()]
            for s in range(steps - 1):
                logits.append(ref.forward_batch([[tokens[i][s]] for i in idx]).cpu())
            per_step = torch.stack(logits, dim=1)
            for j, i in enumerate(idx):
                rows[i] = per_step[j]
        out[name] = torch.stack(rows)
        del ref
    return out


def check(product_logits, tokens, variants, label):
    """product_logits [rows, steps, vocab] (the product's bf16 logits as floats), tokens [rows][steps]."""
    tok = torch.tensor(tokens)
    rows, steps = tok.shape
    assert torch.equal(product_logits.argmax(-1), tok), "product tokens are not the argmax of its own logits"
    names = list(variants)
    pair_mismatch, pair_std = {}, {}
    step_diff = torch.zeros(steps)
    for a, b in itertools.combinations(names, 2):
        d = variants[a] - variants[b]
        pair_mismatch[(a, b)] = int((variants[a].argmax(-1) != variants[b].argmax(-1)).sum())
        pair_std[(a, b)] = float(d.std())
        step_diff = torch.maximum(step_diff, d.abs().amax(dim=(0, 2)))
    ref = variants["fp32"]
    ref_tok = ref.argmax(-1)
    diff = product_logits - ref
    mism = (ref_tok != tok).nonzero().tolist()
    details = []
    for r, s in mism:
        margin = float(ref[r, s, ref_tok[r, s]] - ref[r, s, tok[r, s]])
        details.append((r, s, margin, float(step_diff[s])))
    legal = max(pair_mismatch.values())
    bound = legal + 2 * math.sqrt(max(legal, 1))
    stds = list(pair_std.values())
    std_bound = max(stds) + (max(stds) - min(stds))
    prod_std = float(diff.std())
    equal_seqs = int((ref_tok == tok).all(dim=1).sum())
    print(f"[{label}] product vs fp32 oracle: {rows * steps - len(mism)}/{rows * steps} tokens equal, "
          f"{equal_seqs}/{rows} sequences equal over {steps} tokens; mismatches "
          f"{ {'/'.join(k): v for k, v in pair_mismatch.items()} } between legal oracle evaluations "
          f"(bar {len(mism)} <= {bound:.1f}); logit-difference std {prod_std:.5f} (legal "
          f"{min(stds):.5f}..{max(stds):.5f}, bar {std_bound:.5f}); product max logit difference "
          f"{float(diff.abs().max()):.4f}; mismatches (row, step, oracle margin, legal step difference) {details}",
          flush=True)
    assert len(mism) <= bound, (len(mism), bound)
    assert all(margin <= legal_diff for _, _, margin, legal_diff in details), details
    assert prod_std <= std_bound, (prod_std, std_bound)
    return len(mism), legal, equal_seqs
