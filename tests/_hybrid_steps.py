"""Whole-step comparison of a hybrid decode engine with its oracle, shared by the
C4 and C5 engine tests.

The engine runs greedy and records its logits and, per layer, the experts its
router picked.  The oracle replays the same token stream (teacher-forced on the
engine's picks) and follows the engine's routing where the two differ by a
near-tie: an expert swapped in or out within the oracle's slack (bf16 ulps of its
k-th router logit; two by default), which another f32 summation order may settle
either way.  Any other difference in routing fails.  With routing followed, every step's logits
must be within *bound* of max |logit|, and the greedy pick must be equal wherever
the oracle's top-2 margin exceeds twice the step's error."""
import torch


def feed_of(eng, prompts, steps):
    """The engine's input token per sequence and step: the prompt while it lasts,
    then its own pick of the step before (recorded in eng.sam)."""
    sam = eng.sam.cpu()
    return [list(p) + sam[b, len(p) - 1:steps].tolist() for b, p in enumerate(prompts)]


def check_steps(orc, step, logits, routes, feed, prompts, bound):
    """*step(t, tokens, routes)* runs the oracle's step t.  -> (router decisions
    followed at near-ties, greedy picks checked, worst relative error)."""
    rows, steps = len(prompts), logits.shape[0]
    assert routes is not None and routes.shape[0] == steps
    followed = picks = 0
    worst = widest = 0.0
    for t in range(steps):
        want = step(t, [feed[b][t] for b in range(rows)], routes[t])
        got = logits[t]
        err = (got - want).abs().max(dim=1).values
        scale = want.abs().max(dim=1).values
        rel = err / scale
        fol, far, dist = orc.route_followed[-1], orc.route_far[-1], orc.route_dist[-1]
        print(f"step {t}: rel err {[round(v, 5) for v in rel.tolist()]} "
              f"routes followed {fol.tolist()}", flush=True)
        assert not far.any(), ("routing differs past a near-tie", t, far.tolist(),
                               "swap distance in ulps of the k-th logit", dist.tolist())
        widest = max(widest, float(dist.max()))
        assert (err <= bound * scale).all(), (t, rel.tolist(), bound)
        followed += int(fol.sum())
        worst = max(worst, float(rel.max()))
        top2 = want.topk(2, dim=1).values
        for b in range(rows):
            if t >= len(prompts[b]) - 1 and top2[b, 0] - top2[b, 1] > 2 * err[b]:
                picks += 1
                assert int(got[b].argmax()) == int(want[b].argmax()), (t, b)
                assert feed[b][t + 1] == int(want[b].argmax()), (t, b)
    print(f"router decisions followed at near-ties: {followed} of "
          f"{rows * steps * routes.shape[1]} (row, step, layer), the widest {widest:g} ulps; "
          f"greedy picks checked {picks}; worst rel err {worst:.4f} (bound {bound})", flush=True)
    return followed, picks, worst
