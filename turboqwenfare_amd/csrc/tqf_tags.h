// tqf_tags.h -- the tags of the persistent stack kernel's partial words.
//
// Phase C publishes each member's partial rows as 64-bit words
// (tag << 32 | f32 bits), and the members of a team poll the words until
// they carry the tag of the current (launch, layer).  A word therefore must
// never still hold the current tag from an earlier launch or layer.
//
// The tags count layer steps: the sync block holds `base`, the number of
// layer steps all earlier launches on that scratch have run (mod 2^31); a
// launch of n layers tags layer l with base + l and, at its exit, advances
// base by n.  Tags are strictly increasing (mod 2^31) over the whole launch
// sequence whatever the depth of each launch, so the word a launch reads was
// last written either by this launch or with an earlier tag, which differs
// from the current one unless 2^31 layer steps passed in between; every word
// is rewritten at every layer of every launch, so at most one launch's
// layers lie in between.
//
// Plain constexpr functions: device code and the host-side test of the tag
// sequence (tests/test_stack_tags.py) compile the same definitions.
#pragma once

#include <stdint.h>

namespace tqf {

// The tag of layer l of a launch whose first layer step is `base`; the high
// bit is always set, so a zeroed word never matches.
constexpr uint32_t stack_part_tag(uint32_t base, uint32_t l) {
    return 0x80000000u | ((base + l) & 0x7FFFFFFFu);
}

// The base of the launch after one of n_layers layers (wraps mod 2^31).
constexpr uint32_t stack_next_base(uint32_t base, uint32_t n_layers) {
    return (base + n_layers) & 0x7FFFFFFFu;
}

}  // namespace tqf
