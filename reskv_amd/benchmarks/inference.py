"""Time greedy decoding of a local Llama checkpoint with the ResKV cache or with
dense KV, and write one JSON report.  ``python -m reskv_amd.benchmarks.inference
--model <dir> --method reskv|dense ...`` (the reference's benchmarks/inference.py
command line)."""

import argparse
from pathlib import Path

import torch

from .common import check_run, declare_run, kernel_config_for, prompt_ids, require_gpu, save_json
from .timing import repeated_runs, run_header


def _parse():
    parser = argparse.ArgumentParser(description=__doc__)
    declare_run(parser)
    parser.add_argument("--method", choices=["reskv", "dense"], default="reskv")
    parser.add_argument("--output", type=Path, default=Path("results/inference.json"))
    args = parser.parse_args()
    check_run(parser, args)
    if args.method == "reskv" and args.dtype != "fp16":
        parser.error("ResKV inference requires --dtype fp16")
    require_gpu(parser)
    config = None
    if args.method == "reskv":
        try:
            config = kernel_config_for(args)
            config.resolve(args.batch_size)
        except ValueError as exc:
            parser.error(str(exc))
    return parser, args, config


def _load_model(parser, args, config):
    import transformers

    model_config = transformers.AutoConfig.from_pretrained(args.model)
    if model_config.model_type != "llama":
        parser.error("performance benchmarks support Llama checkpoints only")
    options = {"config": model_config, "attn_implementation": "sdpa",
               "dtype": torch.float16 if args.dtype == "fp16" else torch.bfloat16}
    if config is None:
        return transformers.LlamaForCausalLM.from_pretrained(args.model, **options)
    from ..models.llama import ResKVForCausalLM

    return ResKVForCausalLM.from_pretrained(args.model, kernel_config=config, **options)


def main():
    import transformers

    parser, args, config = _parse()
    torch.manual_seed(args.seed)
    model = _load_model(parser, args, config).cuda().eval()
    ids, digest = prompt_ids(model.config.vocab_size, args.batch_size, args.input_length, args.seed)
    records = repeated_runs(model, ids, args, dense=config is None)
    report = {**run_header(args, digest, transformers.__version__), "method": args.method, "model_dtype": args.dtype,
              "kernel_config": None if config is None else config.to_dict(),
              "kernel_plan": None if config is None else config.resolve(args.batch_size).to_dict(),
              "records": records}
    print(save_json(args.output, report), end="")


if __name__ == "__main__":
    main()
