"""Writes tests/golden/decoder_kats.json: the reference's own known-answer cases for the
decoder-layer operators, as numbers.

Each case is one test of the reference's suite, with its inputs and attributes exactly as
the test builds them and its expected outputs computed from the test's own closed form or
inline reference, restated here in float64:

  FusedLlmNormTests.cs:47-131        RmsNorm_LastAxis_HandComputed, RmsNorm_Scale_And_InvStdOutput,
                                     SkipRmsNorm_SumThenNorm_HandComputed, SkipRmsNorm_WithBiasBetaGamma
                                     (expected values: the hand formulas in each test)
  GqaGenaiTests.cs:45-420            PackedQkv_NoRotary_MatchesUnpackedAndReference,
                                     PackedQkv_Rotary_HalfSplit_MatchesManual,
                                     Rotary_Interleaved_vs_HalfSplit_Differ, Decode_WithPast_AndSeqlensK,
                                     SeqlensK_BoundsKeyRange, Unpacked_NoRotary_Unchanged
                                     (RefCausal :45-72, RotHalf :75-86, RotInterleaved :89-100)
  GqaSlidingWindowTests.cs:46-240    Window2_SingleHead_AttendsSelfPlusOnePrevious,
                                     WindowDisabledOrLarge_EqualsFullCausal, Window1_AttendsSelfOnly,
                                     DecodeWithPast_WindowExcludesOldCachedKeys (RefWindow :49-80)

The reference tests compare at an absolute 1e-4; so do the tests that read this file. Run
from the repository root: python tests/golden/make_decoder_kats.py
"""
from __future__ import annotations

import json
import pathlib

import numpy as np

OUT = pathlib.Path(__file__).resolve().parent / "decoder_kats.json"


def ref_window(q, k, v, scale, past_offset, window):
    """RefWindow (GqaSlidingWindowTests.cs:49-80); window < 0 is RefCausal (GqaGenaiTests.cs:45-72).
    q [Sq, hd], k/v [Sk, hd]; query i (absolute past_offset + i) sees keys
    [max(0, qAbs - window + 1), min(qAbs, Sk - 1)]."""
    q, k, v = (np.asarray(x, np.float64) for x in (q, k, v))
    sq, sk = q.shape[0], k.shape[0]
    out = np.zeros((sq, v.shape[1]))
    for i in range(sq):
        qa = past_offset + i
        lo = max(0, qa - window + 1) if window >= 0 else 0
        hi = min(qa, sk - 1)
        s = np.array([q[i] @ k[j] * scale for j in range(lo, hi + 1)])
        p = np.exp(s - s.max())
        p /= p.sum()
        out[i] = p @ v[lo:hi + 1]
    return out


def rot_half(x, c, s):
    """RotHalf (GqaGenaiTests.cs:75-86): NeoX half-split rotary of one vector."""
    x = np.asarray(x, np.float64)
    h = len(x) // 2
    y = x.copy()
    for j in range(h):
        a, b = x[j], x[j + h]
        y[j] = a * c[j] - b * s[j]
        y[j + h] = b * c[j] + a * s[j]
    return y


def rot_interleaved(x, c, s):
    """RotInterleaved (GqaGenaiTests.cs:89-100): GPT-J pairwise rotary of one vector."""
    x = np.asarray(x, np.float64)
    y = x.copy()
    for j in range(len(x) // 2):
        a, b = x[2 * j], x[2 * j + 1]
        y[2 * j] = a * c[j] - b * s[j]
        y[2 * j + 1] = b * c[j] + a * s[j]
    return y


def per_head(q, k, v, s, H, KH, D, scale, past_offset=0, window=-1):
    """Unpacked [S, H*D] queries over [Sk, KH*D] keys/values, head h on kv head h // (H/KH)."""
    q = np.asarray(q, np.float64).reshape(s, H, D)
    k = np.asarray(k, np.float64).reshape(-1, KH, D)
    v = np.asarray(v, np.float64).reshape(-1, KH, D)
    out = np.zeros((s, H, D))
    for h in range(H):
        kh = h // (H // KH)
        out[:, h] = ref_window(q[:, h], k[:, kh], v[:, kh], scale, past_offset, window)
    return out.reshape(-1)


def gqa_case(name, source, inputs, attrs, expected, **extra):
    return {"op": "GroupQueryAttention", "name": name, "source": source, "inputs": inputs, "attrs": attrs,
            "expected": {k: np.asarray(v, np.float64).ravel().tolist() for k, v in expected.items()}, **extra}


def tensor(shape, data, dtype="float32"):
    return {"shape": list(shape), "dtype": dtype, "data": list(np.asarray(data, np.float64).ravel())}


def norm_cases():
    cases = []
    x = np.array([1, 2, 3, 4.0])
    inv = 1 / np.sqrt(7.5)
    cases.append({"op": "SimplifiedLayerNormalization", "name": "RmsNorm_LastAxis_HandComputed",
                  "source": "FusedLlmNormTests.cs:47-61",
                  "inputs": {"x": tensor([1, 4], x), "scale": tensor([4], [1, 1, 1, 1])}, "attrs": {"epsilon": 0.0},
                  "expected": {"y": (x * inv).tolist()}})
    eps = np.float32(1e-5)
    inv0 = 1 / np.sqrt((9 + 16) / 2 + float(eps))
    inv1 = 1 / np.sqrt((1 + 1) / 2 + float(eps))
    cases.append({"op": "SimplifiedLayerNormalization", "name": "RmsNorm_Scale_And_InvStdOutput",
                  "source": "FusedLlmNormTests.cs:63-84",
                  "inputs": {"x": tensor([2, 2], [3, 4, 1, 1]), "scale": tensor([2], [2, 0.5])},
                  "attrs": {"epsilon": float(eps)},
                  "expected": {"y": [3 * inv0 * 2, 4 * inv0 * 0.5, 1 * inv1 * 2, 1 * inv1 * 0.5], "inv": [inv0, inv1]}})
    t = np.array([2, 4, 3, 4.0])
    inv = 1 / np.sqrt(11.25)
    cases.append({"op": "SkipSimplifiedLayerNormalization", "name": "SkipRmsNorm_SumThenNorm_HandComputed",
                  "source": "FusedLlmNormTests.cs:88-108",
                  "inputs": {"input": tensor([1, 4], [1, 2, 3, 4]), "skip": tensor([1, 4], [1, 2, 0, 0]),
                             "gamma": tensor([4], [1, 1, 1, 1])}, "attrs": {"epsilon": 0.0},
                  "expected": {"out": (t * inv).tolist(), "sum": t.tolist()}})
    inv = 1 / np.sqrt(10.0)
    cases.append({"op": "SkipSimplifiedLayerNormalization", "name": "SkipRmsNorm_WithBiasBetaGamma",
                  "source": "FusedLlmNormTests.cs:110-131",
                  "inputs": {"input": tensor([1, 2], [1, 2]), "skip": tensor([1, 2], [0, 1]),
                             "gamma": tensor([2], [2, 3]), "beta": tensor([2], [0.1, -0.2]),
                             "bias": tensor([2], [1, 1])}, "attrs": {"epsilon": 0.0},
                  "expected": {"out": [2 * inv * 2 + 0.1, 4 * inv * 3 - 0.2]}})
    return cases


def gqa_genai_cases():
    cases = []
    # PackedQkv_NoRotary_MatchesUnpackedAndReference (GqaGenaiTests.cs:106-163)
    packed = [1, 0, 0, 1, 1, 0, 2, 3, 0, 1, 1, 0, 0, 1, 5, 7]
    q = [1, 0, 0, 1, 0, 1, 1, 0]
    k = [1, 0, 0, 1]
    v = [2, 3, 5, 7]
    exp = per_head(q, k, v, 2, 2, 1, 2, 1 / np.sqrt(2))
    cases.append(gqa_case("PackedQkv_NoRotary_MatchesUnpackedAndReference", "GqaGenaiTests.cs:106-163",
                          {"q": tensor([1, 2, 8], packed)}, {"num_heads": 2, "kv_num_heads": 1}, {"out": exp},
                          present_shape=[1, 1, 2, 2]))
    cases.append(gqa_case("PackedQkv_NoRotary_MatchesUnpackedAndReference/unpacked", "GqaGenaiTests.cs:135-143",
                          {"q": tensor([1, 2, 4], q), "k": tensor([1, 2, 2], k), "v": tensor([1, 2, 2], v)},
                          {"num_heads": 2, "kv_num_heads": 1}, {"out": exp}))
    # PackedQkv_Rotary_HalfSplit_MatchesManual (:169-216)
    q0, k0, v0 = [1, 2, 3, 4], [1, 0, 1, 0], [1, 1, 1, 1]
    q1, k1, v1 = [0, 1, 0, 1], [2, 1, 0, 1], [2, 2, 2, 2]
    cos, sin = [1, 1, 0.6, 0.8], [0, 0, 0.8, 0.6]
    c0, s0, c1, s1 = [1, 1], [0, 0], [0.6, 0.8], [0.8, 0.6]

    def rot_ref(rot, q0, k0, v0, q1, k1, v1):
        qh = np.stack([rot(q0, c0, s0), rot(q1, c1, s1)])
        kh = np.stack([rot(k0, c0, s0), rot(k1, c1, s1)])
        return ref_window(qh, kh, np.array([v0, v1], np.float64), 1 / np.sqrt(4), 0, -1)

    packed = q0 + k0 + v0 + q1 + k1 + v1
    cases.append(gqa_case("PackedQkv_Rotary_HalfSplit_MatchesManual", "GqaGenaiTests.cs:169-216",
                          {"q": tensor([1, 2, 12], packed), "cos": tensor([2, 2], cos), "sin": tensor([2, 2], sin)},
                          {"num_heads": 1, "kv_num_heads": 1, "do_rotary": 1},
                          {"out": rot_ref(rot_half, q0, k0, v0, q1, k1, v1)}))
    # Rotary_Interleaved_vs_HalfSplit_Differ (:222-282)
    q0, k0, v0 = [1, 2, 3, 4], [1, 1, 1, 1], [1, 0, 0, 0]
    q1, k1, v1 = [4, 3, 2, 1], [1, 2, 3, 4], [0, 1, 0, 0]
    packed = q0 + k0 + v0 + q1 + k1 + v1
    for inter, rot in ((0, rot_half), (1, rot_interleaved)):
        cases.append(gqa_case(f"Rotary_Interleaved_vs_HalfSplit_Differ/interleaved={inter}", "GqaGenaiTests.cs:222-282",
                              {"q": tensor([1, 2, 12], packed), "cos": tensor([2, 2], cos), "sin": tensor([2, 2], sin)},
                              {"num_heads": 1, "kv_num_heads": 1, "do_rotary": 1, "rotary_interleaved": inter},
                              {"out": rot_ref(rot, q0, k0, v0, q1, k1, v1)}))
    # Decode_WithPast_AndSeqlensK (:288-340)
    q = [1, 0, 0, 1]
    k_all = [[1, 0], [0, 1], [1, 1]]
    v_all = [[2, 0], [0, 4], [9, 9]]
    exp = per_head(q, k_all, v_all, 1, 2, 1, 2, 1 / np.sqrt(2), past_offset=2)
    cases.append(gqa_case("Decode_WithPast_AndSeqlensK", "GqaGenaiTests.cs:288-340",
                          {"q": tensor([1, 1, 4], q), "k": tensor([1, 1, 2], [1, 1]), "v": tensor([1, 1, 2], [9, 9]),
                           "past_key": tensor([1, 1, 2, 2], [1, 0, 0, 1]),
                           "past_value": tensor([1, 1, 2, 2], [2, 0, 0, 4]),
                           "seqlens_k": tensor([1], [2], "int32")},
                          {"num_heads": 2, "kv_num_heads": 1},
                          {"out": exp, "present_key": np.array(k_all)}, present_shape=[1, 1, 3, 2]))
    # SeqlensK_BoundsKeyRange (:346-363)
    cases.append(gqa_case("SeqlensK_BoundsKeyRange", "GqaGenaiTests.cs:346-363",
                          {"q": tensor([1, 2, 1], [1, 1]), "k": tensor([1, 2, 1], [0.5, 0.5]),
                           "v": tensor([1, 2, 1], [3, 9]), "seqlens_k": tensor([1], [0], "int32")},
                          {"num_heads": 1, "kv_num_heads": 1}, {"out": [3, 3]}))
    # Unpacked_NoRotary_Unchanged (:369-381): pos0 sees key0 only, pos1 equal scores
    cases.append(gqa_case("Unpacked_NoRotary_Unchanged", "GqaGenaiTests.cs:369-381",
                          {"q": tensor([1, 2, 2], [1, 1, 1, 1]), "k": tensor([1, 2, 1], [0.5, 0.5]),
                           "v": tensor([1, 2, 1], [3, 9])},
                          {"num_heads": 2, "kv_num_heads": 1}, {"out": [3, 3, 6, 6]}))
    return cases


def gqa_window_cases():
    cases = []
    # Window2_SingleHead_AttendsSelfPlusOnePrevious (GqaSlidingWindowTests.cs:110-140)
    q = [0.3, 0.7, 1.1, 0.2, 0.9]
    k = [0.5, 0.2, 0.8, 0.4, 0.6]
    v = [1, 2, 3, 4, 5]
    exp = ref_window(np.array(q)[:, None], np.array(k)[:, None], np.array(v)[:, None], 1.0, 0, 2)
    cases.append(gqa_case("Window2_SingleHead_AttendsSelfPlusOnePrevious", "GqaSlidingWindowTests.cs:110-140",
                          {"q": tensor([1, 5, 1], q), "k": tensor([1, 5, 1], k), "v": tensor([1, 5, 1], v)},
                          {"num_heads": 1, "kv_num_heads": 1, "local_window_size": 2}, {"out": exp},
                          bounds=[[1, 1], [1, 2], [2, 3]]))
    # WindowDisabledOrLarge_EqualsFullCausal (:146-185)
    q = [1, 0, 0, 1, 0.5, 0.5, 1, 1, 0.2, 0.9, 0.7, 0.3, 1, 0.4, 0.6, 0.8]
    k = [1, 0, 0, 1, 0.5, 0.5, 0.3, 0.9]
    v = [2, 3, 5, 7, 1, 1, 4, 8]
    exp = per_head(q, k, v, 4, 2, 1, 2, 1 / np.sqrt(2))
    for w in (-1, 100):
        cases.append(gqa_case(f"WindowDisabledOrLarge_EqualsFullCausal/window={w}", "GqaSlidingWindowTests.cs:146-185",
                              {"q": tensor([1, 4, 4], q), "k": tensor([1, 4, 2], k), "v": tensor([1, 4, 2], v)},
                              {"num_heads": 2, "kv_num_heads": 1, "local_window_size": w}, {"out": exp}))
    # Window1_AttendsSelfOnly (:191-203)
    cases.append(gqa_case("Window1_AttendsSelfOnly", "GqaSlidingWindowTests.cs:191-203",
                          {"q": tensor([1, 4, 1], [0.3, 0.7, 1.1, 0.2]), "k": tensor([1, 4, 1], [0.5, 0.2, 0.8, 0.4]),
                           "v": tensor([1, 4, 1], [1, 2, 3, 4])},
                          {"num_heads": 1, "kv_num_heads": 1, "local_window_size": 1}, {"out": [1, 2, 3, 4]}))
    # DecodeWithPast_WindowExcludesOldCachedKeys (:209-245)
    k_all = [[5, 5], [6, 6], [0, 1], [1, 1]]
    v_all = [[100, 100], [200, 200], [3, 4], [9, 9]]
    exp = ref_window(np.array([[1.0, 0.0]]), np.array(k_all, np.float64), np.array(v_all, np.float64),
                     1 / np.sqrt(2), 3, 2)
    cases.append(gqa_case("DecodeWithPast_WindowExcludesOldCachedKeys", "GqaSlidingWindowTests.cs:209-245",
                          {"q": tensor([1, 1, 2], [1, 0]), "k": tensor([1, 1, 2], [1, 1]), "v": tensor([1, 1, 2], [9, 9]),
                           "past_key": tensor([1, 1, 3, 2], [5, 5, 6, 6, 0, 1]),
                           "past_value": tensor([1, 1, 3, 2], [100, 100, 200, 200, 3, 4]),
                           "seqlens_k": tensor([1], [3], "int32")},
                          {"num_heads": 1, "kv_num_heads": 1, "local_window_size": 2}, {"out": exp},
                          below=10.0))
    return cases


def main():
    cases = norm_cases() + gqa_genai_cases() + gqa_window_cases()
    OUT.write_text(json.dumps({"tolerance": 1e-4, "cases": cases}, indent=1) + "\n")
    print(f"wrote {len(cases)} cases to {OUT}")


if __name__ == "__main__":
    main()
