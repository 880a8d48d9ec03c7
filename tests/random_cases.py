"""Seeded random configurations across the argument space of the eight ops.

Each case is a tests/golden/cases.py case dict (so `make_inputs` builds its
tensors): odd oversampling factors including < 1, cutoffs from 0 to beyond
the box, reconstruction boxes other than the backprojection size, batch and
pose broadcasting, absent shifts / weights / gradient inputs, both dtypes and
interpolations, and pose matrices that are not rotations.
"""
import random

from tests.golden.cases import BPBACK, BPFORW, FORW, PBACK, _case

OPS = FORW + PBACK + BPFORW + BPBACK


def random_cases(count, seed, max_n=40, min_p=1):
    rng = random.Random(seed)
    out = []
    for k in range(count):
        op = OPS[k % len(OPS)]
        n = 2 * rng.randint(1, max_n // 2)
        os_ = rng.choice([0.5, 0.75, 1.0, 1.25, 1.5, 2.0, 2.5, 3.0])
        cut = rng.choice([None, None, 0.0, round(rng.uniform(0.5, n), 3), 1000.0])
        B = rng.randint(1, 3)
        rec_n = None
        if op in FORW + PBACK and rng.random() < 0.3:
            rec_n = 2 * rng.randint(1, max(1, int(n * os_)))
        c = _case(f"rand{seed}_{k}_{op}", op, dtype="f64" if rng.random() < 0.2 else "f32",
                  interp=rng.choice(["linear", "cubic"]), os=os_, cutoff=cut, B=B,
                  P=rng.choice([min_p, 1, 2, 5, 13]), n=n, rec_n=rec_n, shifts=rng.random() < 0.7,
                  B_rot=rng.choice([1, B]), B_shift=rng.choice([1, B]), weights=rng.random() < 0.6,
                  grad_weight_rec=rng.random() < 0.6, rg_rot=rng.random() < 0.6, rg_sh=rng.random() < 0.6,
                  special=rng.random() < 0.3, seed=rng.randint(0, 2 ** 31 - 1))
        c["scaled"] = rng.random() < 0.25  # turn every other pose matrix into a scaled one
        out.append(c)
    return out


def binned_cases():
    """The 3D scatters with enough poses for the per-call pose bins (16 or more): a rotation per
    batch item (B_rot = 2, one set of bin lists each) or broadcast, both interpolations, every other
    pose scaled in the per-item cases (the bins also serve the kernels of other tiled poses)."""
    rng = random.Random(9090)
    out = []
    seed = 9090
    for op in ("backproject_2d_to_3d_forw", "project_3d_to_2d_back"):
        for interp in ("linear", "cubic"):
            for B_rot in (1, 2):
                seed += 1
                c = _case(f"binned_{op}_{interp}_brot{B_rot}", op, interp=interp,
                          os=rng.choice([1.0, 1.5, 2.0]), cutoff=rng.choice([None, 9.5]), B=2,
                          P=rng.choice([16, 40, 70]), n=2 * rng.randint(8, 18), B_rot=B_rot, B_shift=2, seed=seed)
                c["scaled"] = B_rot == 2
                out.append(c)
    return out


def many_pose_cases():
    """66000 poses in one call (small projections): past the 65536 poses from which the 3D scatters
    go without pose bins (their list entries are 16-bit) and past any 16-bit pose index, in the
    forward, both 3D scatters and the 2D scatter."""
    out = []
    seed = 7070
    for op, interp in (("project_3d_to_2d_forw", "linear"), ("backproject_2d_to_3d_forw", "linear"),
                       ("backproject_2d_to_3d_forw", "cubic"), ("project_3d_to_2d_back", "linear"),
                       ("backproject_2d_forw", "linear")):
        seed += 1
        out.append(_case(f"many_{op}_{interp}", op, interp=interp, os=2.0, B=1, P=66000, n=8, seed=seed,
                         rg_rot=False, rg_sh=False))
        out[-1]["scaled"] = False
    return out


def large_shift_cases():
    """Shifts of a few hundred pixels (N(0, 500^2)): phase angles r s0 + c s1 up to ~1e5 rad, whose
    fp32 value the reference rounds before its sine and cosine, for every op with a phase."""
    out = []
    seed = 8080
    for op in OPS:
        for interp in ("linear", "cubic"):
            seed += 1
            out.append(_case(f"bigshift_{op}_{interp}", op, interp=interp, os=2.0, B=1, P=7, n=32, seed=seed,
                             shift_scale=500.0))
            out[-1]["scaled"] = False
    return out


def reflect_poses(args, case):
    """Negate column 0 of every other pose matrix: orthonormal columns with determinant -1 (a
    reflection), which the tiled kernels take as they take rotations."""
    idx = {"project_3d_to_2d_forw": 1, "project_2d_forw": 1, "project_3d_to_2d_back": 2, "project_2d_back": 2,
           "backproject_2d_to_3d_forw": 2, "backproject_2d_forw": 2,
           "backproject_2d_to_3d_back": 4, "backproject_2d_back": 4}[case["op"]]
    rot = args[idx]
    rg = rot.requires_grad
    r = rot.detach().clone()
    r[:, ::2, :, 0] *= -1
    args[idx] = r.requires_grad_(rg)
    return args


def reflect_cases():
    """Every op, both interpolations, with every other pose a reflection (reflect_poses)."""
    rng = random.Random(9191)
    out = []
    seed = 9191
    for op in OPS:
        for interp in ("linear", "cubic"):
            seed += 1
            c = _case(f"reflect_{op}_{interp}", op, interp=interp, os=rng.choice([1.0, 1.5, 2.0]), B=2, P=6,
                      n=2 * rng.randint(6, 16), B_rot=rng.choice([1, 2]), seed=seed)
            c["scaled"] = False
            c["reflect"] = True
            out.append(c)
    return out


def odd_cases():
    """Odd projection sizes n (rows i <= n // 2 are frequencies 0..m, the others -m..-1 for
    n = 2m + 1: one more negative row than an even size has), every op, both interpolations, with
    and without a cutoff, every other case's pose matrices scaled."""
    rng = random.Random(6060)
    out = []
    seed = 6060
    for op in OPS:
        for interp in ("linear", "cubic"):
            seed += 1
            n = rng.choice([9, 15, 21, 33])
            c = _case(f"odd_{op}_{interp}_n{n}", op, interp=interp, os=rng.choice([1.0, 1.5, 2.0]),
                      cutoff=rng.choice([None, round(rng.uniform(2.0, n / 2), 3)]), B=2, P=5, n=n,
                      B_rot=rng.choice([1, 2]), seed=seed)
            c["scaled"] = interp == "cubic"
            out.append(c)
    return out


def scale_poses(args, case):
    """Scale every other pose matrix by 1.05 (a matrix that is not a rotation)."""
    idx = {"project_3d_to_2d_forw": 1, "project_2d_forw": 1, "project_3d_to_2d_back": 2, "project_2d_back": 2,
           "backproject_2d_to_3d_forw": 2, "backproject_2d_forw": 2,
           "backproject_2d_to_3d_back": 4, "backproject_2d_back": 4}[case["op"]]
    rot = args[idx]
    rg = rot.requires_grad
    r = rot.detach().clone()
    r[:, ::2] *= 1.05
    args[idx] = r.requires_grad_(rg)
    return args


def nonfinite_cutoff_cases():
    """Every op with a radius cutoff of +inf, NaN, 3e9 (a square beyond every int) and 1e30 (whose fp32
    square overflows): the mask keeps every pixel (r^2 + c^2 > inf and > NaN are false), so the
    results equal those without a cutoff but wider than the grid."""
    out = []
    seed = 5150
    for op in OPS:
        for tag, cut in (("inf", float("inf")), ("nan", float("nan")), ("3e9", 3e9), ("1e30", 1e30)):
            seed += 1
            interp = "cubic" if tag == "nan" else "linear"
            n = 32 if "3d" in op else 48
            c = _case(f"cut{tag}_{op}_{interp}", op, interp=interp, os=2.0, cutoff=cut, B=1, P=6, n=n, seed=seed)
            c["scaled"] = False
            out.append(c)
    return out
