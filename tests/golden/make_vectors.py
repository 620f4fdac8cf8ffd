"""Writes known_answers.json: inputs whose expected outputs follow from the
definitions by hand, not from the oracle.

- quantize: groups whose peak is 127 (so the scale is exactly 1 and each
  code is the input rounded half to even, clamped to +-127), and groups
  whose peak is 254 (scale 2: codes are x/2 rounded half to even).
- f16: values on both sides of rounding ties and the subnormal and
  overflow edges, with their IEEE binary16 bit patterns worked out by hand.
- q8_0: blocks with peak 127 (d = 1: codes round half away from zero).
"""

import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    q = []
    x = [127.0, 63.5, 62.5, -0.5, 0.5, 1.5, 2.5, -2.5, -126.5, -127.0, 3.25, -3.75] + [0.0] * 20
    q.append(dict(name="peak127", group=32, half=False, x=x,
                  codes=[127, 64, 62, 0, 0, 2, 2, -2, -126, -127, 3, -4] + [0] * 20, scales=[1.0]))
    x2 = [254.0, 5.0, 3.0, -1.0, 1.0, 7.0, -9.0] + [0.0] * 25
    q.append(dict(name="peak254", group=32, half=False, x=x2,
                  codes=[127, 2, 2, 0, 0, 4, -4] + [0] * 25, scales=[2.0]))
    q.append(dict(name="zeros", group=32, half=True, x=[0.0] * 32, codes=[0] * 32, scales=[1.0]))
    f16 = [
        dict(value=1.0, bits=0x3C00), dict(value=-2.0, bits=0xC000), dict(value=65504.0, bits=0x7BFF),
        dict(value=65520.0, bits=0x7C00),            # rounds up to infinity
        dict(value=2.0 ** -24, bits=0x0001),          # smallest subnormal
        dict(value=2.0 ** -25, bits=0x0000),          # tie to even: 0
        dict(value=3 * 2.0 ** -25, bits=0x0002),      # tie to even: 2 * 2^-24
        dict(value=1 + 2.0 ** -11, bits=0x3C00),      # tie to even: 1.0
        dict(value=1 + 3 * 2.0 ** -11, bits=0x3C02),  # tie to even: 1 + 2^-9
        dict(value=2.0 ** -14, bits=0x0400),          # smallest normal
    ]
    q80 = [dict(name="d1", x=[127.0, 0.5, -0.5, 1.5, 2.5, -2.5, 3.25, -126.5] + [0.0] * 24,
                codes=[127, 1, -1, 2, 3, -3, 3, -127] + [0] * 24, scales=[1.0])]
    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump(dict(quantize=q, f16=f16, q8_0=q80), f, indent=1)


if __name__ == "__main__":
    main()
