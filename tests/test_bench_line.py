"""bench.py's stdout line: short enough for the driver to parse, with the contract's keys.

The full result (every kernel's figures, the linear stack, the other configs) is large;
bench.py writes it to stderr and a side file and prints only compact_result() of it.
These tests build a full result of the real shape from canned numbers (no GPU) and check
the line's size and keys.
"""
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402

UNITS = ["embed_rows", "embed_ln", "qkv.quant", "qkv.gemm", "attention", "o.quant", "o.gemm", "attn_ln+quant",
         "ffn_up.gemm", "ffn_down.quant", "ffn_down.gemm", "out_ln+quant", "out_ln", "pool"]


def canned_result(n_units: int = len(UNITS), long_notes: bool = True) -> dict:
    note = "x" * (600 if long_notes else 10)
    units = {}
    for i in range(n_units):
        label = UNITS[i % len(UNITS)] + ("" if i < len(UNITS) else f"#{i}")
        u = {"launches_per_step": 12.0, "us_per_launch": 100.0 + i, "us_per_launch_median": 99.0,
             "us_per_launch_min": 90.0, "us_per_launch_max": 120.0, "ops": 1.5e11 if "gemm" in label else 0.0,
             "bytes": 4.3e8, "kind": "w8a8", "kernel": "enchip::gemm_w8a8_pt<128, 256, 64, 2, 2, true, 4, 0>",
             "ms_per_step": 1.2, "alg_gbps": 2400.0, "frac_hbm_peak": 0.3}
        if u["ops"]:
            u.update(int8_tops=870.0, frac_int8_peak=0.17)
        if label == "attention":
            u["frac_mfma_peak"] = 0.37
        units[label] = u
    other = {f"cfg{i}": {"us_per_call": 1.0, "note": note, "kernels": {str(j): note for j in range(5)}}
             for i in range(9)}
    other["config2_isolated_linear"] = {"us_per_call": 39.7, "note": note}
    other["config3_gemv_n768"] = {"us_per_call": 5.78, "frac_hbm_peak": 0.0155, "note": note}
    other["config3_gemv_n3072"] = {"us_per_call": 5.86, "frac_hbm_peak": 0.0566, "note": note}
    other["rerank_device_cfg5"] = {"pairs_per_s": 2443.6, "note": note}
    other["ann_flat_i8_m1"] = {"us_per_call": 59.2, "note": note}
    other["ffn_gelu_placement"] = {str(sd): {"gemm_gelu_us": 189.7, "quant_us": 82.1, "gemm_bias_us": 118.6,
                                             "gelu_quant_us": 131.9, "epilogue_pair_us": 271.8123,
                                             "quantizer_pair_us": 250.5123, "tails": 0.0113, "codes_identical": True}
                                   for sd in (0.28, 0.55, 1.1, 3.3)}
    other["ffn_gelu_placement"]["note"] = note
    return {
        "metric": bench.METRIC, "value": 7227.6123456, "unit": "seqs/s", "n_gpus": 1, "steps": 20, "warmup": 3,
        "ms_per_step": 8.8551234, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic",
        "config": {"workload": note, "model": "bert-base (random-init weights, per-channel int8)",
                   "global_batch": 64, "seq_len": 512, "tokens_per_step": 32768, "parallelism": "single GPU",
                   "attention_products": "split-bf16 online-softmax (ENCHIP_ATT_FLASH_BF16)",
                   "seeds": {"weights": 2024}, "launch": "eager"},
        "output_finite": True,
        "encode_kernels": units,
        "encode_kernels_timing": note,
        "roofline": {"bound": "hbm", "achieved": 2427.8383, "peak": 8000.0, "unit": "GB/s", "frac": 0.30348,
                     "traffic": 449113736, "kernel": "enchip::gemm_w8a8_pt<128, 256, 64, 2, 2, true, 4, 0>",
                     "unit_label": "ffn_up.gemm", "avg_launch_us": 177.25, "alg_bytes_per_launch": 430333952.0,
                     "alg_ops_per_launch": 154618822656.0, "limiter": note, "scope": note,
                     "traffic_source": bench.TRAFFIC_PROFILE,
                     "valu": {"lane_ops_per_output": 36, "outputs_per_launch": 100663296,
                              "lane_ops_per_launch": 3.6e9, "achieved_t_lane_ops": 20.4,
                              "measured_peak_t_lane_ops": 60.1, "frac": 0.34}},
        "roofline_step_dominant": {"unit_label": "ffn_up.gemm", "kernel": "k", "avg_launch_us": 177.25,
                                   "launches_per_step": 12.0, "share_of_step": 0.23, "bound": "hbm",
                                   "unit": "GB/s", "achieved": 2427.8, "peak": 8000.0, "frac": 0.3035,
                                   "valu_frac": 0.34},
        "measured_ceilings": {"hbm_read_gbps": 7186.1, "hbm_write_gbps": 5201.9, "mfma_i8_tops": 4287.7,
                              "valu_f32_tops": 60.1, "mfma_i8_mhz": 2102.2, "mfma_i8_data_tops": 3285.7,
                              "mfma_i8_data_mhz": 1615.0},
        "linear_stack": {"ms_per_step": 5.81, "kernels": {str(i): note for i in range(20)}, "note": note},
        "other_configs": other,
        "encode_f32_products": {"ms_per_step": 15.57, "note": note},
        "cpu_baseline": {"value": 2.156, "unit": "seqs/s", "cores": 16, "kind": "port", "sample": note,
                         "ms_per_layer": {"linears": 25.6}},
    }


REQUIRED = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
            "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline")


def test_line_is_short_and_keeps_the_contract_keys():
    full = canned_result()
    assert len(json.dumps(full)) > 20000  # the shape that the driver could not parse
    line = bench.compact_result(full, "gpurun_out/bench_detail.json")
    text = json.dumps(line, allow_nan=False)
    assert len(text) <= 4096, len(text)
    assert "\n" not in text
    for k in REQUIRED:
        assert k in line, k
    assert line["value"] == full["value"] or abs(line["value"] - full["value"]) < 1e-2
    for k in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert k in line["roofline"], k
    assert line["roofline"]["valu"]["frac"] == 0.34
    for k in ("value", "unit", "cores", "kind", "sample"):
        assert k in line["cpu_baseline"], k
    assert line["kernels_us_frac"]["ffn_up.gemm"] == [108.0, 0.17]
    assert line["kernels_us_frac"]["attention"][1] == 0.37
    assert line["other"]["cfg5_pairs_per_s"] == 2444.0
    assert line["other"]["ffn_gelu_epi_vs_quant_us"]["0.55"] == [271.8, 250.5, 0.0113]
    assert line["measured_ceilings"]["mfma_i8_tops"] == 4288.0
    assert json.loads(text) == line


def test_line_stays_under_the_limit_with_many_kernels():
    line = bench.compact_result(canned_result(n_units=400))
    assert len(json.dumps(line)) <= bench.LINE_LIMIT
    for k in REQUIRED:
        assert k in line, k


def test_line_without_cpu_baseline_or_other_configs():
    full = canned_result()
    full["cpu_baseline"] = None
    del full["other_configs"], full["linear_stack"]
    line = bench.compact_result(full)
    assert line["cpu_baseline"] is None
    assert "cfg5_pairs_per_s" not in line["other"]
    assert len(json.dumps(line)) <= 4096


def test_line_with_the_gelu_quantizer_dominant():
    # FFN-up's GELU applied by FFN-down's quantizer: the W8A8 path's dominant kernel is then
    # the quantizer, whose binding roof is VALU issue; the line keeps its valu roof, and
    # its measured traffic comes from the traffic profile's gelu_quant row.
    full = canned_result()
    units = full["encode_kernels"]
    units["ffn_down.gelu_quant"] = dict(units["ffn_down.quant"], kernel="enchip::quant_rows_frag_gelu<12>",
                                        us_per_launch=118.8)
    del units["ffn_down.quant"]
    full["roofline"] = {"bound": "hbm", "achieved": 4237.0, "peak": 8000.0, "unit": "GB/s", "frac": 0.5297,
                        "traffic": bench.measured_traffic().get(bench.traffic_key_of("ffn_down.gelu_quant")),
                        "kernel": "enchip::quant_rows_frag_gelu<12>", "unit_label": "ffn_down.gelu_quant",
                        "avg_launch_us": 118.8, "alg_bytes_per_launch": 503447552.0, "alg_ops_per_launch": 0.0,
                        "limiter": "VALU issue", "scope": "s", "traffic_source": bench.TRAFFIC_PROFILE,
                        "valu": {"lane_ops_per_output": bench.GELU_QUANT_LANE_OPS, "outputs_per_launch": 100663296,
                                 "lane_ops_per_launch": 5.4e9, "achieved_t_lane_ops": 45.8,
                                 "measured_peak_t_lane_ops": 59.7, "frac": 0.767}}
    line = bench.compact_result(full)
    assert len(json.dumps(line, allow_nan=False)) <= 4096
    assert line["roofline"]["unit_label"] == "ffn_down.gelu_quant"
    assert line["roofline"]["valu"]["frac"] == 0.767
    assert line["roofline"]["valu"]["lane_ops_per_output"] == bench.GELU_QUANT_LANE_OPS
    assert line["roofline"]["traffic"] == 503694006  # profiles/bert_base_b64s512_hbm_traffic.md
    assert line["kernels_us_frac"]["ffn_down.gelu_quant"][0] == 118.8


def test_traffic_keys_name_profile_rows():
    assert bench.traffic_key_of("ffn_up.gemm") == "ffn_up"
    assert bench.traffic_key_of("o.quant") == "quant_o"
    assert bench.traffic_key_of("ffn_down.gelu_quant") == "gelu_quant_ffn_down"
    rows = bench.measured_traffic()
    for label in ("qkv.gemm", "o.quant", "o.gemm", "ffn_up.gemm", "ffn_down.gelu_quant", "ffn_down.gemm"):
        assert bench.traffic_key_of(label) in rows, label
