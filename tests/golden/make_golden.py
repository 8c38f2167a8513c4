"""Writes tests/golden/reference_known_answers.json.

Every value below is copied from an assertion or fixture in sungdomo/CastForge's own tests
(cited per entry) or derived by hand from one of them with the arithmetic shown; nothing here
runs or imports the reference.  Run: python tests/golden/make_golden.py
"""
import json
import struct
from pathlib import Path


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


GOLDEN = {
    # src/codegen/config.rs:528-529
    "int_bounds": {"4": [4, -8.0, 7.0], "8": [8, -128.0, 127.0]},
    # tests/ai_opt_tests.rs:656 weight [[0.5,-0.25],[0.75,0.5]] through quantize(bits=8):
    # amax 0.75; f32(0.75/127) = 0.0059055118 (bits 0x3bc18306); v/scale =
    # [84.6667, -42.3333, 127.0, 84.6667] -> round -> [85, -42, 127, 85];
    # "{:.6}" -> "0.005906"; evaluator dequant with the parsed string scale f32(0.005906):
    # q * 0.005906 -> [0.50201, -0.248052, 0.750062, 0.50201].
    "int8_per_tensor": {
        "source": "tests/ai_opt_tests.rs:656",
        "weights": [0.5, -0.25, 0.75, 0.5],
        "codes": [85, -42, 127, 85],
        "scale_bits": 0x3BC18306,
        "scale_string": "0.005906",
        "type_string": "!quant.uniform<i8:f32,0.005906:0>",
        "dequant_with_string_scale": [0.50201, -0.248052, 0.750062, 0.50201],
    },
    # tests/serving_storage_routing_tests.rs:2228-2240 (f32_to_fp8_e4m3fn / fp8_e4m3fn_to_f32)
    "e4m3fn": {
        "encode": [[0.0, 0x00], [-0.0, 0x80], ["nan", 0x7F], [1000.0, 0x7E], [-1000.0, 0xFE]],
        "decode": [[0x7E, 448.0], [0xFE, -448.0], [0x7F, "nan"]],
        "roundtrip": [0.0, 0.125, -0.5, 1.0, 1.5, -3.5, 16.0, 448.0],
    },
    # src/ir/translator.rs:295-296: f32_to_f16_bits(-1e-10) == 0x8000
    "f16_trunc": [[-1e-10, 0x8000]],
    # tests/frontend_tests.rs:747-756: quantize(scheme=awq,bits=4,group_size=2,salient_ratio=0.25)
    # on a 2x2 weight -> castforge.awq_salient_channels = 1 (ceil(f32(4) * 0.25) = 1)
    "awq_salient_count": {"n": 4, "ratio": 0.25, "count": 1},
    # src/codegen/eval.rs:39-44 synthetic inputs ((i*7 + arg*13 + 3) % 19 - 9) * 0.1 for arg 0
    "eval_synthetic_arg0": [((i * 7 + 3) % 19 - 9) * 0.1 for i in range(8)],
}

if __name__ == "__main__":
    out = Path(__file__).with_name("reference_known_answers.json")
    out.write_text(json.dumps(GOLDEN, indent=1, sort_keys=True) + "\n")
    print(out)
