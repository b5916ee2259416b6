"""Writes reference_kats.json: the known-answer tests held by the reference's
own test suite for the hot path, as plain data (inputs and expected outputs).

Every case names the reference test it comes from.  Inputs that the reference
builds from a formula (e.g. ``(i % 7) - 3``) are materialised here; expected
values are the literal numbers the reference asserts.  Cases whose expected
value the reference computes with a JS loop carry ``"expected": null`` and a
``"check"`` describing the closed form the tests evaluate instead.

Run:  python tests/golden/make_kats.py   (rewrites the JSON next to it)
"""
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))


def rng(n, f):
    return [f(i) for i in range(n)]


def conv(args, inp, weight, bias, out_shape, expected, tol, dtype="float32", src=""):
    stride, padding, dilation, transposed, output_padding, groups = args
    return {
        "op": "aten.convolution.default", "dtype": dtype, "source": src,
        "input": inp, "weight": weight, "bias": bias,
        "stride": stride, "padding": padding, "dilation": dilation,
        "transposed": transposed, "output_padding": output_padding, "groups": groups,
        "out_shape": out_shape, "expected": expected, "tol": tol,
    }


def t(shape, data):
    return {"shape": shape, "data": data}


cases = []

# ---- tests/shaders/mm.test.ts
cases.append({"op": "aten.mm.default", "dtype": "float32", "source": "tests/shaders/mm.test.ts:6-22",
              "a": t([2, 2], [1, 2, 3, 4]), "b": t([2, 2], [5, 6, 7, 8]),
              "expected": [19, 22, 43, 50], "tol": 1e-5})
for n, tol, src in ((64, 1e-3, "tests/shaders/mm.test.ts:24-62"),
                    (128, 1e-2, "tests/shaders/mm.test.ts:64-101")):
    cases.append({"op": "aten.mm.default", "dtype": "float32", "source": src,
                  "a": t([n, n], rng(n * n, lambda i: (i % 7) - 3)),
                  "b": t([n, n], rng(n * n, lambda i: (i % 5) - 2)),
                  "expected": None, "check": "exact integer matmul (JS loop in the test)",
                  "tol": tol})
cases.append({"op": "aten.mm.default", "dtype": "float16", "source": "tests/shaders/mm.test.ts:103-122",
              "a": t([2, 2], [1, 2, 3, 4]), "b": t([2, 2], [5, 6, 7, 8]),
              "expected": [19, 22, 43, 50], "tol": 0.05})
cases.append({"op": "aten.mm.default", "dtype": "float16", "source": "tests/shaders/mm.test.ts:124-162",
              "a": t([64, 64], rng(64 * 64, lambda i: (i % 7) - 3)),
              "b": t([64, 64], rng(64 * 64, lambda i: (i % 5) - 2)),
              "expected": None, "check": "exact integer matmul (JS loop in the test)", "tol": 0.5})
cases.append({"op": "aten.mm.default", "dtype": "float32", "source": "tests/shaders/mm.test.ts:164-196",
              "a": t([5, 7], rng(35, lambda i: (i % 5) - 2)),
              "b": t([7, 3], rng(21, lambda i: (i % 3) + 1)),
              "expected": None, "check": "exact integer matmul (JS loop in the test)", "tol": 1e-4})

# ---- tests/shaders/bmm.test.ts
cases.append({"op": "aten.bmm.default", "dtype": "float32", "source": "tests/shaders/bmm.test.ts:6-23",
              "a": t([1, 2, 3], [1, 2, 3, 4, 5, 6]), "b": t([1, 3, 2], [7, 8, 9, 10, 11, 12]),
              "expected": [58, 64, 139, 154], "tol": 1e-3})
cases.append({"op": "aten.bmm.default", "dtype": "float32", "source": "tests/shaders/bmm.test.ts:25-41",
              "a": t([2, 2, 2], [1, 0, 0, 1, 2, 0, 0, 3]), "b": t([2, 2, 2], [5, 6, 7, 8, 5, 6, 7, 8]),
              "expected": [5, 6, 7, 8, 10, 12, 21, 24], "tol": 1e-3})
cases.append({"op": "aten.bmm.default", "dtype": "float16", "source": "tests/shaders/bmm.test.ts:43-66",
              "a": t([2, 2, 2], [1, 0, 0, 1, 2, 0, 0, 3]), "b": t([2, 2, 2], [5, 6, 7, 8, 5, 6, 7, 8]),
              "expected": [5, 6, 7, 8, 10, 12, 21, 24], "tol": 0.05})
ident = [0.0] * (2 * 64 * 64)
bdat = [0.0] * (2 * 64 * 64)
for bb in range(2):
    for i in range(64):
        ident[bb * 4096 + i * 64 + i] = 1.0
        for j in range(64):
            bdat[bb * 4096 + i * 64 + j] = (i + j) * 0.1
cases.append({"op": "aten.bmm.default", "dtype": "float32", "source": "tests/shaders/bmm.test.ts:68-100",
              "a": t([2, 64, 64], ident), "b": t([2, 64, 64], bdat),
              "expected": None, "check": "identity: out == b (toBeCloseTo 3 digits)", "tol": 5e-4})

# ---- tests/shaders/convolution.test.ts
S = "tests/shaders/convolution.test.ts"
cases.append(conv(([1, 1], [0, 0], [1, 1], False, [0, 0], 1),
                  t([1, 1, 3, 3], [1, 2, 3, 4, 5, 6, 7, 8, 9]), t([1, 1, 2, 2], [1, 0, 0, 1]),
                  t([1], [10]), [1, 1, 2, 2], [16, 18, 22, 24], 1e-5, src=S + ":6-45"))
cases.append(conv(([1, 1], [0, 0], [1, 1], False, [0, 0], 2),
                  t([1, 2, 2, 2], [1, 2, 3, 4, 10, 20, 30, 40]),
                  t([2, 1, 2, 2], [1, 1, 1, 1, 1, 0, 0, 1]), None, [1, 2, 1, 1], [10, 50], 1e-5,
                  src=S + ":47-92"))
cases.append(conv(([2, 2], [0, 0], [1, 1], True, [0, 0], 1),
                  t([1, 1, 2, 2], [1, 2, 3, 4]), t([1, 1, 2, 2], [1, 1, 1, 1]), None, [1, 1, 4, 4],
                  [1, 1, 2, 2, 1, 1, 2, 2, 3, 3, 4, 4, 3, 3, 4, 4], 1e-5, src=S + ":94-130"))
cases.append(conv(([2, 2], [1, 1], [1, 1], False, [0, 0], 1),
                  t([1, 2, 5, 5], rng(50, lambda i: i + 1)),
                  t([3, 2, 3, 3], rng(54, lambda i: (i + 1) * 0.1)),
                  t([3], [2.5, -1.0, 0.5]), [1, 3, 3, 3],
                  [202.5, 312.9, 214.5, 370.3, 559.0, 373.9, 264.9, 392.1, 257.7, 436.6, 698.2,
                   491.8, 885.2, 1381.7, 953.6, 715.0, 1101.4, 751.0, 675.7, 1088.5, 774.1, 1405.1,
                   2209.4, 1538.3, 1170.1, 1815.7, 1249.3], 1e-3, src=S + ":132-176"))
cases.append(conv(([2, 2], [1, 1], [1, 1], True, [1, 1], 1),
                  t([1, 2, 3, 3], rng(18, lambda i: i + 1)),
                  t([2, 2, 3, 3], rng(36, lambda i: (i + 1) * 0.05)),
                  t([2], [1.5, -2.0]), [1, 2, 6, 6],
                  [13.25, 26.3, 14.65, 29.1, 16.05, 16.8, 28.3, 57.7, 31.1, 63.3, 33.9, 35.7, 17.45,
                   34.7, 18.85, 37.5, 20.25, 21.3, 36.7, 74.5, 39.5, 80.1, 42.3, 44.7, 21.65, 43.1,
                   23.05, 45.9, 24.45, 25.8, 25.1, 50.3, 26.8, 53.7, 28.5, 29.85,
                   14.7, 33.6, 17.0, 38.2, 19.3, 20.05, 37.4, 81.2, 42.0, 90.4, 46.6, 48.4, 21.6, 47.4,
                   23.9, 52.0, 26.2, 27.25, 51.2, 108.8, 55.8, 118.0, 60.4, 62.8, 28.5, 61.2, 30.8,
                   65.8, 33.1, 34.45, 31.95, 68.4, 34.55, 73.6, 37.15, 38.5], 1e-5,
                  src=S + ":178-225"))
cases.append(conv(([1, 1], [0, 0], [1, 1], False, [0, 0], 1),
                  t([1, 1, 3, 3], [1, 2, 3, 4, 5, 6, 7, 8, 9]), t([1, 1, 2, 2], [1, 0, 0, 1]),
                  t([1], [10]), [1, 1, 2, 2], [16, 18, 22, 24], 1e-2, dtype="float16",
                  src=S + ":227-256"))
cases.append(conv(([1, 1], [0, 0], [1, 1], False, [0, 0], 1),
                  t([1, 64, 8, 8], rng(64 * 64, lambda i: ((i % 5) - 2) * 0.5)),
                  t([64, 64, 1, 1], rng(64 * 64, lambda i: ((i % 7) - 3) * 0.25)),
                  None, [1, 64, 8, 8], None, 0.05, dtype="float16", src=S + ":258-306"))
cases[-1]["check"] = "element 0 = sum_ic in[ic*64] * w[ic] (toBeCloseTo 1 digit)"
cases.append(conv(([1, 1], [0, 0], [1, 1], False, [0, 0], 2),
                  t([1, 2, 2, 2], [1, 2, 3, 4, 10, 20, 30, 40]), t([2, 1, 1, 1], [2, 0.5]),
                  None, [1, 2, 2, 2], [2, 4, 6, 8, 5, 10, 15, 20], 1e-2, dtype="float16",
                  src=S + ":308-336"))
w1x1 = [0.0] * 16
for o in range(4):
    w1x1[o * 4 + o] = 2.0
cases.append(conv(([1, 1], [0, 0], [1, 1], False, [0, 0], 1),
                  t([1, 4, 2, 2], rng(16, lambda i: i + 1)), t([4, 4, 1, 1], w1x1), None,
                  [1, 4, 2, 2], rng(16, lambda i: 2 * (i + 1)), 5e-5, src=S + ":338-380"))
cases.append(conv(([1, 1], [0, 0], [1, 1], False, [0, 0], 1),
                  t([1, 16, 8, 8], rng(16 * 64, lambda i: (i % 13) * 0.1)),
                  t([64, 16, 1, 1], rng(64 * 16, lambda i: (i % 7) * 0.1)), None,
                  [1, 64, 8, 8], None, 5e-4, src=S + ":382-420"))
cases[-1]["check"] = "element 0 = sum_c in[c*64] * w[c] (toBeCloseTo 3 digits)"
cases.append(conv(([1, 1], [0, 0], [1, 1], False, [0, 0], 2),
                  t([1, 4, 2, 2], [1.0] * 16), t([4, 2, 1, 1], [2.0] * 8), None, [1, 4, 2, 2],
                  [4.0] * 16, 1e-3, src=S + ":422-449"))

# ---- tests/api/program.test.ts: out = (a + 1.5 b) @ c
cases.append({"op": "program", "source": "tests/api/program.test.ts:25-68",
              "a": [1, 2, 3, 4], "b": [10, 20, 30, 40], "c": [1, 2, 3, 4], "alpha": 1.5,
              "expected": [112, 160, 240, 352], "tol": 1e-5})

with open(os.path.join(HERE, "reference_kats.json"), "w") as f:
    json.dump({"about": "known-answer tests transcribed from the reference test suite",
               "cases": cases}, f, indent=0)
print(f"wrote {len(cases)} cases")
