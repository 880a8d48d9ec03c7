"""Case table and input construction for the golden vectors (tests/golden/*.npz).

`CASES` lists one dict per fixture; `make_inputs(case)` draws the seeded input
tensors and `build_args(case, tensors)` turns named tensors into the
positional argument list of the dispatcher op (csrc/torch_projectors.cpp:23-36).
The replay tests load the stored tensors and call `build_args`, so fixtures do
not depend on the RNG of a particular torch version.
"""
import math

import torch

# ops whose first argument is a reconstruction (forward family) vs projections
FORW = ("project_2d_forw", "project_3d_to_2d_forw")
PBACK = ("project_2d_back", "project_3d_to_2d_back")
BPFORW = ("backproject_2d_forw", "backproject_2d_to_3d_forw")
BPBACK = ("backproject_2d_back", "backproject_2d_to_3d_back")


TAGS = {"project_2d_forw": "p2_forw", "project_3d_to_2d_forw": "p3_forw", "project_2d_back": "p2_back",
        "project_3d_to_2d_back": "p3_back", "backproject_2d_forw": "bp2_forw",
        "backproject_2d_to_3d_forw": "bp3_forw", "backproject_2d_back": "bp2_back",
        "backproject_2d_to_3d_back": "bp3_back"}


def is_3d(op):
    return "3d" in op


def rec_boxsize(n, os_):
    raw = int(math.ceil(n * os_))
    return raw + raw % 2


def rotations_3d(P, gen, dtype, special=False):
    q = torch.randn(P, 4, generator=gen, dtype=torch.float64)
    q = q / q.norm(dim=1, keepdim=True)
    w, x, y, z = q.unbind(1)
    R = torch.stack([1 - 2 * (y * y + z * z), 2 * (x * y - z * w), 2 * (x * z + y * w),
                     2 * (x * y + z * w), 1 - 2 * (x * x + z * z), 2 * (y * z - x * w),
                     2 * (x * z - y * w), 2 * (y * z + x * w), 1 - 2 * (x * x + y * y)], 1).reshape(P, 3, 3)
    if special and P >= 2:
        R[0] = torch.eye(3, dtype=torch.float64)
        R[1] = torch.tensor([[0., -1., 0.], [1., 0., 0.], [0., 0., 1.]], dtype=torch.float64)
    return R.to(dtype)


def rotations_2d(P, gen, dtype, special=False):
    a = torch.rand(P, generator=gen, dtype=torch.float64) * 2 * math.pi
    if special and P >= 2:
        a[0] = 0.0
        a[1] = math.pi / 2
    c, s = torch.cos(a), torch.sin(a)
    return torch.stack([c, -s, s, c], 1).reshape(P, 2, 2).to(dtype)


def _case(name, op, **kw):
    d = dict(name=name, op=op, dtype="f32", interp="linear", os=1.0, cutoff=None, B=2, P=3, n=8,
             rec_n=None, shifts=True, B_rot=None, B_shift=None, weights=True, grad_weight_rec=True,
             rg_rot=True, rg_sh=True, special=False, seed=0, rec_kind="randn")
    d.update(kw)
    if d["B_rot"] is None:
        d["B_rot"] = d["B"]
    if d["B_shift"] is None:
        d["B_shift"] = d["B"]
    return d


def _cases():
    out = []
    seed = 1000
    for op in FORW + PBACK + BPFORW + BPBACK:
        tag = TAGS[op]
        for interp in ("linear", "cubic"):
            for os_, cut in ((1.0, None), (2.0, None), (1.5, 3.0)):
                seed += 1
                out.append(_case(f"{tag}_{interp}_os{os_:g}", op, interp=interp, os=os_, cutoff=cut, seed=seed,
                                 special=(os_ == 1.0)))
        # broadcast rotations/shifts, no shifts, no weights / no grad_weight_rec, f64
        seed += 1
        out.append(_case(f"{tag}_linear_bcast_noshift", op, os=2.0, B_rot=1, shifts=False, weights=False,
                         grad_weight_rec=False, rg_rot=False, seed=seed))
        seed += 1
        out.append(_case(f"{tag}_cubic_bcast", op, interp="cubic", os=2.0, B_rot=1, B_shift=1, rg_sh=False,
                         grad_weight_rec=False, seed=seed))
        seed += 1
        out.append(_case(f"{tag}_f64_cubic", op, dtype="f64", interp="cubic", os=2.0, B=1, seed=seed))
        if op in FORW + PBACK:
            # projection box larger than the reconstruction box reaches the clamped edge
            seed += 1
            out.append(_case(f"{tag}_linear_edge", op, os=1.0, n=12, rec_n=8, seed=seed, cutoff=9.0))
            seed += 1
            out.append(_case(f"{tag}_cubic_edge", op, interp="cubic", os=1.0, n=12, rec_n=8, seed=seed,
                             cutoff=9.0))
        if op in FORW:
            seed += 1
            out.append(_case(f"{tag}_linear_impulse", op, os=2.0, P=4, special=True, rec_kind="impulse",
                             shifts=False, seed=seed))
    return out


CASES = _cases()


def make_inputs(case):
    """Draw the seeded inputs of `case`; returns (args, tensors)."""
    g = torch.Generator().manual_seed(case["seed"])
    cdt = torch.complex64 if case["dtype"] == "f32" else torch.complex128
    rdt = torch.float32 if case["dtype"] == "f32" else torch.float64
    op, B, P, n = case["op"], case["B"], case["P"], case["n"]
    three = is_3d(op)
    rot_fn = rotations_3d if three else rotations_2d
    R = torch.stack([rot_fn(P, g, rdt, case["special"]) for _ in range(case["B_rot"])])
    sh = (torch.randn(case["B_shift"], P, 2, generator=g, dtype=torch.float64) * case.get("shift_scale", 2.5)).to(rdt) \
        if case["shifts"] else None
    t = {"rotations": R, "shifts": sh}
    if op in FORW + PBACK:
        N = case["rec_n"] or rec_boxsize(n, case["os"])
        shape = (B, N, N, N // 2 + 1) if three else (B, N, N // 2 + 1)
        if case["rec_kind"] == "impulse":
            rec = torch.zeros(shape, dtype=cdt)
            idx = [torch.randint(0, s, (5,), generator=g) for s in shape]
            rec[tuple(idx)] = torch.randn(5, generator=g, dtype=cdt)
        else:
            rec = torch.randn(shape, generator=g, dtype=cdt)
        t["reconstruction"] = rec
        if op in PBACK:
            t["grad_projections"] = torch.randn(B, P, n, n // 2 + 1, generator=g, dtype=cdt)
    else:
        t["projections"] = torch.randn(B, P, n, n // 2 + 1, generator=g, dtype=cdt)
        t["weights"] = torch.rand(B, P, n, n // 2 + 1, generator=g, dtype=rdt) if case["weights"] else None
        if op in BPBACK:
            N = rec_boxsize(n, case["os"])
            shape = (B, N, N, N // 2 + 1) if three else (B, N, N // 2 + 1)
            t["grad_data_rec"] = torch.randn(shape, generator=g, dtype=cdt)
            t["grad_weight_rec"] = torch.randn(shape, generator=g, dtype=rdt) if case["grad_weight_rec"] else None
    return build_args(case, t), t


def build_args(case, t):
    """Positional arguments of the dispatcher op from named tensors."""
    op = case["op"]
    rot = t["rotations"].clone().requires_grad_(bool(case["rg_rot"]) and op in PBACK + BPBACK)
    sh = t.get("shifts")
    if sh is not None:
        sh = sh.clone().requires_grad_(bool(case["rg_sh"]) and op in PBACK + BPBACK)
    tail = [case["interp"], float(case["os"]), case["cutoff"]]
    if op in FORW:
        return [t["reconstruction"], rot, sh, [case["n"], case["n"]], *tail]
    if op in PBACK:
        return [t["grad_projections"], t["reconstruction"], rot, sh, *tail]
    if op in BPFORW:
        return [t["projections"], t.get("weights"), rot, sh, *tail]
    return [t["grad_data_rec"], t.get("grad_weight_rec"), t["projections"], t.get("weights"), rot, sh, *tail]
