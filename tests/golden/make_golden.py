"""Write tests/golden/readout_cases.json: known-answer vectors for the readout.

The reference ships no golden vectors (it checks against its eager oracle on
random data), so these are computed here from first principles, independently
of torch and of the oracle under test:
  * forward by plain Python loops in fp64 with a max-shifted log-sum-exp;
  * gradients from the hand-derived backward (docs/DESIGN.md:26-37 of the
    reference):  dS = P * (gO E^T - delta),  delta = rowsum(O * gO) - glse,
    gh = s dS W, gW = s dS^T h, gE = P^T gO, gb = colsum(dS);
  * every gradient entry is checked here against a central finite difference
    of the scalar L = sum(gO * O) + sum(glse * lse) before it is written;
  * MSE loss values (swvr/api.py:53-66) for each reduction.
Inputs come from Python's `random` with fixed seeds; the file is committed.

    python tests/golden/make_golden.py
"""
import json
import math
import os
import random

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "readout_cases.json")


def forward(h, W, E, b, s):
    N, V, D = len(h), len(W), len(E[0]) if E else 0
    O, lse, P = [], [], []
    for n in range(N):
        S = [s * sum(hk * wk for hk, wk in zip(h[n], W[v])) + (b[v] if b is not None else 0.0) for v in range(V)]
        m = max(S)
        shift = 0.0 if m == -math.inf else m
        z = sum(math.exp(x - shift) for x in S)
        ls = shift + math.log(z)
        p = [math.exp(x - ls) for x in S]
        P.append(p)
        lse.append(ls)
        O.append([sum(p[v] * E[v][d] for v in range(V)) for d in range(D)])
    return O, lse, P


def backward(h, W, E, b, s, gO, glse):
    N, K, V, D = len(h), len(h[0]), len(W), len(E[0])
    O, lse, P = forward(h, W, E, b, s)
    delta = [sum(O[n][d] * gO[n][d] for d in range(D)) - glse[n] for n in range(N)]
    dS = [[P[n][v] * (sum(gO[n][d] * E[v][d] for d in range(D)) - delta[n]) for v in range(V)] for n in range(N)]
    gh = [[s * sum(dS[n][v] * W[v][k] for v in range(V)) for k in range(K)] for n in range(N)]
    gW = [[s * sum(dS[n][v] * h[n][k] for n in range(N)) for k in range(K)] for v in range(V)]
    gE = [[sum(P[n][v] * gO[n][d] for n in range(N)) for d in range(D)] for v in range(V)]
    gb = [sum(dS[n][v] for n in range(N)) for v in range(V)]
    return gh, gW, gE, gb


def objective(h, W, E, b, s, gO, glse):
    O, lse, _ = forward(h, W, E, b, s)
    return sum(gO[n][d] * O[n][d] for n in range(len(O)) for d in range(len(O[0]))) + \
        sum(g * x for g, x in zip(glse, lse))


def finite_difference_check(h, W, E, b, s, gO, glse, grads, eps=1e-6, tol=1e-6):
    names = ["h", "W", "E", "b"]
    mats = [h, W, E, b]
    for name, mat, g in zip(names, mats, grads):
        if mat is None:
            continue
        rows = mat if isinstance(mat[0], list) else [mat]
        grows = g if isinstance(g[0], list) else [g]
        for i, row in enumerate(rows):
            for j in range(len(row)):
                x0 = row[j]
                if not math.isfinite(x0):
                    continue
                row[j] = x0 + eps
                fp = objective(h, W, E, b, s, gO, glse)
                row[j] = x0 - eps
                fm = objective(h, W, E, b, s, gO, glse)
                row[j] = x0
                fd = (fp - fm) / (2 * eps)
                an = grows[i][j]
                assert abs(fd - an) <= tol * max(1.0, abs(an)), (name, i, j, fd, an)


def mse(O, lse, target, weight, reduction, z):
    per = [sum((o - t) ** 2 for o, t in zip(O[n], target[n])) / len(O[n]) + z * lse[n] ** 2 for n in range(len(O))]
    if weight is not None:
        per = [p * w for p, w in zip(per, weight)]
    if reduction == "none":
        return per
    if reduction == "sum":
        return sum(per)
    return sum(per) / (sum(weight) if weight is not None else len(per))


def rand_mat(rng, r, c, std=1.0):
    return [[rng.gauss(0.0, std) for _ in range(c)] for _ in range(r)]


def make_case(name, seed, N, K, V, D, bias=True, scale=1.0, edit_bias=None, fd=True):
    rng = random.Random(seed)
    h = rand_mat(rng, N, K)
    W = rand_mat(rng, V, K, 1.0 / math.sqrt(K))
    E = rand_mat(rng, V, D)
    b = [rng.gauss(0.0, 0.5) for _ in range(V)] if bias else None
    if edit_bias:
        for v, x in edit_bias.items():
            b[v] = x
    gO = rand_mat(rng, N, D)
    glse = [rng.gauss(0.0, 1.0) for _ in range(N)]
    O, lse, _ = forward(h, W, E, b, scale)
    grads = backward(h, W, E, b, scale, gO, glse)
    if fd:
        finite_difference_check(h, W, E, b, scale, gO, glse, grads)
    gh, gW, gE, gb = grads
    return dict(name=name, N=N, K=K, V=V, D=D, logit_scale=scale, h=h, W=W, E=E, bias=b, gO=gO, glse=glse,
                O=O, lse=lse, gh=gh, gW=gW, gE=gE, gb=gb if bias else None)


def main():
    cases = [
        make_case("basic", 1, N=3, K=4, V=5, D=2, scale=0.7),
        make_case("no_bias", 2, N=2, K=3, V=7, D=3, bias=False),
        make_case("single_vocab", 3, N=3, K=4, V=1, D=3),
        make_case("masked_vocab", 4, N=3, K=4, V=6, D=2, edit_bias={0: -math.inf, 4: -math.inf}),
        # bias +-1e4: the softmax is one-hot on row 2 to fp64 precision; finite
        # differences through exp(-1e4) are meaningless, so only the closed form
        make_case("dominant_bias", 5, N=2, K=3, V=5, D=2, edit_bias={2: 1e4, 3: -1e4}, fd=False),
        make_case("wide", 6, N=5, K=9, V=11, D=4, scale=2.5),
    ]
    # MSE loss on one case, every reduction (swvr/api.py:53-66)
    rng = random.Random(7)
    c = make_case("mse", 8, N=4, K=3, V=5, D=2, scale=0.5)
    target = rand_mat(rng, 4, 2)
    weight = [1.0, 0.0, 2.0, 0.5]
    z = 0.1
    c["target"], c["weight"], c["z_loss_weight"] = target, weight, z
    c["mse"] = {red: mse(c["O"], c["lse"], target, weight, red, z) for red in ("mean", "sum", "none")}
    c["mse_unweighted_mean"] = mse(c["O"], c["lse"], target, None, "mean", z)
    cases.append(c)
    with open(OUT, "w") as f:
        json.dump({"generator": "tests/golden/make_golden.py", "cases": cases}, f, indent=None)
        f.write("\n")
    print(f"wrote {OUT}: {len(cases)} cases")


if __name__ == "__main__":
    main()
