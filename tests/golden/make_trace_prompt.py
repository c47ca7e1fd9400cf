"""Writes tiny_gemma_dev/trace_prompt.json: the prompt of the reference's
golden checkpoint traces (tests/golden_traces.rs:68, LONG_PROMPT) and its token
ids.

prompt_prepare (routines/prompt_prepare/native/tiles.rs) renders the chat
template `{% for message in messages %}{{ message.content }}{% endfor %}`
(the prompt unchanged) and encodes it with tokenizer.json and
add_special_tokens (the template processor adds nothing). The ids are
computed here with the `tokenizers` library on the fixture tokenizer.json;
the prompt.prepare entry of traces/native-det-full.json pins them (it is the
SHA-256 of a payload holding the ids and their digest). Run from the
repository root: python tests/golden/make_trace_prompt.py
"""
import json
import pathlib

from tokenizers import Tokenizer

HERE = pathlib.Path(__file__).resolve().parent
PROMPT = "hello raster prompt"


def main() -> None:
    tok = Tokenizer.from_file(str(HERE / "tiny_gemma_dev" / "tokenizer.json"))
    ids = tok.encode(PROMPT, add_special_tokens=True).ids
    out = {"prompt_text": PROMPT, "prompt_token_ids": ids}
    (HERE / "tiny_gemma_dev" / "trace_prompt.json").write_text(json.dumps(out, indent=1) + "\n")
    print(out)


if __name__ == "__main__":
    main()
