"""Text in, text out: the token loop of predict_token_by_token
(network_types/transformer/transformer_network.rs:165-313) around the
network's cached predict, whose forward passes run on the device.

What the reference does around the forward pass, restated here:
  - every input is prefixed with "<bos> " (network_components/input.rs:70-72);
  - it is tokenized with the GPT-NeoX tokenizer, special tokens added
    (utils/tokenizer.rs:9-41; tokenize_batch(.., with_eos = false));
  - at most MAX_CONTEXT_WINDOW_SIZE ids are kept, the last ones
    (transformer_network.rs:32, 208-218);
  - step 0 runs every prompt row; later steps feed the last id at
    time_step = its position (:225-248, 300-304);
  - each step's whole output is kept (:257: [S][V] Re-logits at step 0, then
    [1][V]) and the greedy id is taken from the last row (:258-263,
    sampling_methods.rs:5-18: the last index among equal maxima, NaN is an
    error), decoded on its own with special tokens kept (utils/tokenizer.rs:43-50);
  - a token that decodes to "<eos>" ends the loop without being appended
    (:285-288); any other token's text is appended to sequence 0's text (:291);
  - the loop ends after 21 appended tokens (:293-297).

Only sequence 0 is continued (batch_ids[0].push, :266), so the loop is the
reference's batch-1 path: sequence 0 is generated and the other texts are
returned with their "<bos> " prefix and nothing appended.  The tokenizer is
passed in (any object with the `tokenizers.Tokenizer` encode/decode calls);
the reference loads it from TOKENIZER_GPT_NEOX_PATH, relative to its crate root.
"""
from __future__ import annotations

import numpy as np

MAX_CONTEXT_WINDOW_SIZE = 512  # transformer_network.rs:32
MAX_NEW_TOKENS = 21            # count_tokens_prediction > 20 ends the loop (:293-297)
EOS_TEXT = "<eos>"             # :285
BOS_PREFIX = "<bos> "          # input.rs:70-72
TOKENIZER_GPT_NEOX_PATH = "src/neural_networks/tokenizers/gtp_neox_tokenizer.json"  # utils/tokenizer.rs:6


def load_tokenizer(path: str):
    """The tokenizer file the reference reads (Tokenizer::from_file)."""
    from tokenizers import Tokenizer

    return Tokenizer.from_file(path)


def greedy_id(row) -> int:
    """greedy_decoding of one row (sampling_methods.rs:5-18): max_by keeps the
    last of equal maxima; a NaN makes partial_cmp().unwrap() panic."""
    row = np.asarray(row, dtype=np.float64)
    if np.isnan(row).any():
        raise ValueError("greedy_decoding: NaN in logits (sampling_methods.rs:12)")
    return int(row.shape[0] - 1 - np.argmax(row[::-1]))


def predict_token_by_token(net, input_batch, tokenizer):
    """Greedy continuation of input_batch[0] as text.

    Returns (predictions, texts): `predictions` holds every step's output of
    sequence 0, Re-logits [S][V] at step 0 (every prompt row) and [1][V]
    after; `texts` are the inputs with the "<bos> " prefix, sequence 0
    extended by the generated tokens' text.
    """
    texts = [BOS_PREFIX + t for t in input_batch]
    if not texts:
        return [], texts
    ids = tokenizer.encode(texts[0], add_special_tokens=True).ids[-MAX_CONTEXT_WINDOW_SIZE:]
    if not ids:
        return [], texts
    net.reset()  # a fresh k_cache per call, as predict_by_text reloads the model (:639-652)
    out, _ = net.predict(np.asarray([ids], dtype=np.uint32), forward_only=True)
    predictions = [np.asarray(out[0])]
    pos = len(ids)
    for count in range(MAX_NEW_TOKENS):
        nxt = greedy_id(predictions[-1][-1])
        token = tokenizer.decode([nxt], skip_special_tokens=False)
        if token == EOS_TEXT:
            break
        texts[0] += token
        if count + 1 == MAX_NEW_TOKENS:
            break
        out, _ = net.predict(np.asarray([[nxt]], dtype=np.uint32), time_steps=[pos], forward_only=True)
        predictions.append(np.asarray(out[0]))
        pos += 1
    return predictions, texts
