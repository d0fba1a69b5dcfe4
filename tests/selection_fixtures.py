"""The reference's selection fixture list (verify_selection_flow.py:160-213),
restated with seeded generators: (name, decoded fp16 [B,A,4+nc], max_det,
agnostic, layout, unique)."""
import torch


def _g(seed):
    return torch.Generator().manual_seed(seed)


def predictions(batch, anchors, classes, unique=False, seed=149):
    g = _g(seed)
    boxes = torch.randn(batch, anchors, 4, generator=g).half()
    if unique:
        scores = torch.stack([torch.randperm(anchors * classes, generator=g).reshape(anchors, classes)
                              for _ in range(batch)]).half() / 128
    else:
        scores = torch.randn(batch, anchors, classes, generator=g).sigmoid().half()
    return torch.cat((boxes, scores), -1)


def fixtures(full=True):
    s = 0
    for agnostic in (False, True):
        for layout in ("contiguous", "transposed", "gapped", "expanded"):
            s += 1
            yield f"unique-{layout}-{agnostic}", predictions(2, 17, 7, True, s), 11, agnostic, layout, True
        tied = torch.cat((torch.arange(164).reshape(1, 41, 4).half(), torch.ones(1, 41, 5).half()), -1)
        yield f"all-tied-{agnostic}", tied, 13, agnostic, "transposed", False
        for anchors in (1, 127, 128, 129, 257):
            s += 1
            yield f"boundary-{anchors}-{agnostic}", predictions(3, anchors, 3, seed=s), anchors, agnostic, "contiguous", False
        s += 1
        yield f"large-class-{agnostic}", predictions(1, 3, 1031, seed=s), 2, agnostic, "contiguous", False
        s += 1
        yield f"zero-k-{agnostic}", predictions(2, 17, 3, seed=s), 0, agnostic, "transposed", False
        yield f"zero-anchors-{agnostic}", torch.empty(2, 0, 9).half(), 7, agnostic, "contiguous", False
        yield f"zero-batch-{agnostic}", torch.empty(0, 17, 9).half(), 7, agnostic, "contiguous", False
        s += 1
        yield f"min-k-{agnostic}", predictions(2, 21, 80, seed=s), 300, agnostic, "transposed", False
    duplicate = torch.tensor([[[1, 2, 3, 4, .9, .8, .01], [5, 6, 7, 8, .7, .6, .02],
                               [9, 10, 11, 12, .5, .4, .03]]], dtype=torch.float16)
    yield "duplicate-anchor", duplicate, 2, False, "gapped", True
    special = torch.tensor([0., -0., float("inf"), -float("inf"), float("nan"), 2 ** -24, -2 ** -24],
                           dtype=torch.float16)
    x = special.repeat(51)[:3 * 13 * 9].reshape(3, 13, 9)
    yield "special", x, 9, False, "gapped", False
    yield "special-agnostic", x, 9, True, "transposed", False
    for anchors in (3360, 8400):
        yield f"detection-{anchors}", predictions(1, anchors, 80, seed=anchors), 300, False, "transposed", False
    for k in (511, 512, 513):
        g = _g(k)
        tied = torch.cat((torch.randn(1, 1025, 4, generator=g).half(), torch.ones(1, 1025, 80).half()), -1)
        yield f"prefix-boundary-{k}", tied, k, False, "transposed", False
    for nc in (1, 15, 16, 17, 31, 80, 257):
        yield f"class-block-{nc}", predictions(2, 144, nc, seed=1000 + nc), 129, False, "transposed", False
    for agnostic in (False, True):  # more anchors than one block holds in registers
        yield f"large-anchors-{agnostic}", predictions(1, 40000, 2, seed=41), 300, agnostic, "transposed", False
    # pair selection where most of the K x nc pairs tie the first stage's
    # threshold: every pair (all scores equal), or thousands (five score levels)
    g = _g(77)
    tied = torch.cat((torch.randn(1, 400, 4, generator=g).half(), torch.ones(1, 400, 80).half()), -1)
    yield "tied-pairs", tied, 300, False, "transposed", False
    coarse = torch.randint(0, 5, (1, 1000, 80), generator=g).half() / 4
    yield "coarse-scores", torch.cat((torch.randn(1, 1000, 4, generator=g).half(), coarse), -1), 300, False, \
        "transposed", False
    if full:
        patterns = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.float16)
        x = torch.cat((torch.zeros(1, 128, 4).half(), patterns.reshape(1, 128, 512)), -1)
        yield "all-half-class-blocks", x, 128, False, "transposed", False
        x = torch.cat((torch.zeros(1, 65536, 4).half(), patterns.reshape(1, 65536, 1)), -1)
        yield "all-half-ordered", x, 65536, True, "transposed", False


def backing_and_view(x, layout):
    """(backing tensor, view function) -- verify_selection_flow.py:202-213."""
    b, a, c = x.shape
    if layout == "contiguous":
        return x.contiguous(), lambda base: base
    if layout == "transposed":
        return x.transpose(1, 2).contiguous(), lambda base: base.transpose(1, 2)
    if layout == "expanded":
        return x[:1].contiguous(), lambda base: base.expand(b, -1, -1)
    base = torch.zeros(b + 1, a * 2 + 2, c * 2 + 3, dtype=x.dtype)
    view = lambda backing: backing[1:, 1:1 + 2 * a:2, 1:1 + 2 * c:2]
    view(base).copy_(x)
    return base, view


def c5_selection_input(seed=5, layout="contiguous"):
    """C5: decoded [1,8400,84]: boxes N(0,1)*100, scores U(0,1) [1,8400,80] with
    injected exact ties (>= 5% duplicates, ties at the K=300 cutoff) and NaNs of
    both signs and different payloads."""
    g = _g(seed)
    boxes = (torch.randn(1, 8400, 4, generator=g) * 100).half()
    scores = torch.rand(1, 8400, 80, generator=g).half()
    flat = scores.view(-1)
    n = flat.numel()
    dup_src = torch.randint(0, n, (n // 20,), generator=g)
    dup_dst = torch.randint(0, n, (n // 20,), generator=g)
    flat[dup_dst] = flat[dup_src]
    # ties at the cutoff: copy the 300th best value to 40 other places
    kth = torch.sort(flat.float(), descending=True).values[299].half()
    flat[torch.randint(0, n, (40,), generator=g)] = kth
    nan_bits = torch.tensor([0x7E00, 0xFE00, 0x7C01, 0xFD55, 0x7FFF], dtype=torch.int32).to(torch.int16)
    pos = torch.randint(0, n, (nan_bits.numel() * 4,), generator=g)
    flat.view(torch.int16)[pos] = nan_bits.repeat(4)
    x = torch.cat((boxes, scores), -1)
    return x
